// Software-pipelined, wave-specialised GDN forward for fp16/bf16 inputs,
// chunk size C = 32 (the headline configuration).
//
// The phase-by-phase kernel in gdn_fwd_kernel.h spends a chunk's time in a
// serial sequence load -> gates -> K K^T -> substitution -> W -> scan, all
// behind workgroup barriers.  Only the scan (u = U + W' S, S <- e^{bC} S +
// K^T u~) depends on the previous chunk, so this kernel runs the
// state-independent work of later chunks concurrently with the scan of the
// current one.  A workgroup has 8 waves with fixed roles and exactly one
// barrier per iteration; iteration `it` scans chunk `it` while the other
// roles work ahead:
//
//   role  wave            chunk   work
//   SCAN  0 .. NSW-1      it      U = Tu V, u = U + W' S, o = P u + e^b Q S,
//                                 S <- e^{bC} S + K^T diag(e^{bC-b}) u
//                                 (16 state columns per wave, state in
//                                 accumulator registers for the whole run)
//   L     NSW             it+2    q rows, k^T, v^T, P = e^{b_t-b_j} Q K^T,
//                                 e^b, e^{bC-b} -> "big" slot (j % 3)
//   WV    NSW+1           it+1    W'^T = K^T Tw^T -> W slot (j % 2)
//   E0,E1 NSW+2, NSW+3    it+8    gates + A = beta e^{b_t-b_j} K K^T (t > j)
//                                 -> A slot (j % 6); E_e owns chunks j = e
//                                 (mod 2) and loads them two iterations ahead
//   S0,S1 NSW+4, NSW+5    pairs   forward substitution T = (I+A)^{-1} for two
//                                 chunks at once (lanes 0-31 / 32-63, one
//                                 column per lane), spread over 4 iterations
//                                 (rows [0,16), [16,23), [23,28), [28,32));
//                                 writes Tw = -T diag(beta e^b) (slot j % 4)
//                                 and Tu = T diag(beta) (slot j % 6)
//
// Pair m = (2m, 2m+1) is solved in iterations 2m-6 .. 2m-3 by S_{m%2}.
// Every slot is written in an earlier iteration than any read of it, and is
// not rewritten before its last read (A: written j-8, last read <= j-3;
// Tw: written >= j-4, read j-1; Tu: read j; big: written j-2, read j-1, j;
// W: written j-1, read j).  Global loads are issued one (L) or two (E)
// iterations before use, so their latency overlaps other work.
//
// Registers that a role carries from one iteration to the next (the state,
// the substitution's column, prefetched tiles) share one array, so the
// kernel's register budget is the largest role's, not the sum.

#pragma once

#include "gdn_fwd_kernel.h"

namespace gdn {

namespace pipe {

constexpr int C = 32;
constexpr int kWaves8 = 8;
constexpr int kThreads8 = kWaves8 * 64;
constexpr int NA = 6, NTW = 4, NTU = 6, NBIG = 3, NWS = 2;

template <int K, int BV>
struct alignas(16) Smem {
  static constexpr int SK = K + 8;   // fp16 row stride of [C][K] tiles
  static constexpr int SC = C + 8;   // fp16 row stride of [*][C] tiles
  f16 q[NBIG][C * SK];
  f16 kt[NBIG][K * SC];
  f16 vt[NBIG][BV * SC];
  f16 p[NBIG][C * SC];
  float eb[NBIG][C];
  float ec[NBIG][C];
  f16 w[NWS][C * SK];
  f16 tw[NTW][C * SC];
  f16 tu[NTU][C * SC];
  float a[NA][C * C];
  float ab[NA][C];      // in-chunk cumsum b for the substitution's scaling
  float abeta[NA][C];
};

template <int K, int BV>
constexpr int carry_words() {
  // SCAN: K/16 accumulator tiles; S: C floats; E: k frags + g, beta;
  // L: q and k frags, the v slice, g, beta.
  constexpr int scan = K / 4;
  constexpr int solve = C;
  constexpr int e = 2 * (K / 32) * 4 + 2;
  constexpr int l = 2 * 2 * (K / 32) * 4 + BV / 4 + 2;
  constexpr int m1 = scan > solve ? scan : solve;
  constexpr int m2 = e > l ? e : l;
  return m1 > m2 ? m1 : m2;
}

__device__ __forceinline__ float fexp(float x) {
  // e^x = 2^(x log2 e) on the hardware exp2.
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

__device__ __forceinline__ float raw_to_float(uint32_t raw, int dtype) {
  if (dtype == GDN_DTYPE_F32) return __uint_as_float(raw);
  if (dtype == GDN_DTYPE_F16) {
    const uint16_t h = (uint16_t)raw;
    return (float)__builtin_bit_cast(f16, h);
  }
  return bf16_bits_to_float(raw & 0xffffu);
}

__device__ __forceinline__ uint32_t load_raw(const void* base, int64_t off, int dtype) {
  if (dtype == GDN_DTYPE_F32) return static_cast<const uint32_t*>(base)[off];
  return static_cast<const uint16_t*>(base)[off];
}

// 8 fp16 MFMA operand values from 16 raw input bytes.
template <typename TIn>
__device__ __forceinline__ f16x8 to_f16x8(const uint4& r) {
  f16 x[8];
  InTraits<TIn>::to_op(r, x);
  return f16x8{x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]};
}

__device__ __forceinline__ uint4 cr_get4(const uint32_t* cr, int i) {
  return uint4{cr[4 * i], cr[4 * i + 1], cr[4 * i + 2], cr[4 * i + 3]};
}
__device__ __forceinline__ void cr_set4(uint32_t* cr, int i, const uint4& v) {
  cr[4 * i] = v.x;
  cr[4 * i + 1] = v.y;
  cr[4 * i + 2] = v.z;
  cr[4 * i + 3] = v.w;
}
__device__ __forceinline__ f32x4 cr_getf4(const uint32_t* cr, int i) {
  return f32x4{__uint_as_float(cr[4 * i]), __uint_as_float(cr[4 * i + 1]),
               __uint_as_float(cr[4 * i + 2]), __uint_as_float(cr[4 * i + 3])};
}
__device__ __forceinline__ void cr_setf4(uint32_t* cr, int i, const f32x4& v) {
  cr[4 * i] = __float_as_uint(v[0]);
  cr[4 * i + 1] = __float_as_uint(v[1]);
  cr[4 * i + 2] = __float_as_uint(v[2]);
  cr[4 * i + 3] = __float_as_uint(v[3]);
}

// Inclusive prefix sum over lanes 0..31 (and separately 32..63).
__device__ __forceinline__ float scan32(float x, int lane) {
#pragma unroll
  for (int d = 1; d < 32; d <<= 1) {
    const float y = __shfl_up(x, d, 32);
    if ((lane & 31) >= d) x += y;
  }
  return x;
}

// One 16-byte row fragment (A/B operand, plain layout) of a [*, K] input:
// lane (n, gq) reads row `row`, columns [32 kb + 8 gq, +8).  Rows >= T read 0.
template <typename TIn>
__device__ __forceinline__ uint4 load_frag(const TIn* base, int64_t row_stride, int row, int T,
                                           int col) {
  if (row >= T) return uint4{0u, 0u, 0u, 0u};
  return *reinterpret_cast<const uint4*>(base + (int64_t)row * row_stride + col);
}

// ---------------------------------------------------------------------------

template <typename TIn, int K, int BV>
__global__ __launch_bounds__(kThreads8) void gdn_fwd_pipe_kernel(const KArgs p) {
  using M = Mma<f16>;
  using S = Smem<K, BV>;
  constexpr int SK = S::SK, SC = S::SC;
  constexpr int NSW = BV / 16;
  constexpr int KB = K / 32, KT = K / 16;
  constexpr int NCR = carry_words<K, BV>();
  static_assert(NSW >= 1 && NSW <= 2, "BV must be 16 or 32");
  static_assert(K == 64 || K == 128, "K must be 64 or 128");

  __shared__ S s;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int n = lane & 15;
  const int gq = lane >> 4;

  int unit = blockIdx.x;
  if (p.xcd_remap) unit = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  const int vs = unit % p.nv;
  const int bh = unit / p.nv;
  const int bi = bh / p.H;
  const int hi = bh % p.H;
  const int v0 = vs * BV;
  const int T = p.T;
  const int nch = (T + C - 1) / C;

  const TIn* qg = static_cast<const TIn*>(p.q) + bi * p.sq[0] + hi * p.sq[2];
  const TIn* kg = static_cast<const TIn*>(p.k) + bi * p.sk[0] + hi * p.sk[2];
  const TIn* vg = static_cast<const TIn*>(p.v) + bi * p.sv[0] + hi * p.sv[2] + v0;
  const int64_t g_base = bi * p.sg[0] + hi * p.sg[2];
  const int64_t b_base = bi * p.sb[0] + hi * p.sb[2];
  const int64_t sqt = p.sq[1], skt = p.sk[1], svt = p.sv[1];

  // Role of this wave (wave-uniform).
  enum { R_SCAN, R_L, R_WV, R_E, R_S, R_IDLE };
  int role, ridx;
  if (wave < NSW) {
    role = R_SCAN; ridx = wave;
  } else if (wave == NSW) {
    role = R_L; ridx = 0;
  } else if (wave == NSW + 1) {
    role = R_WV; ridx = 0;
  } else if (wave < NSW + 4) {
    role = R_E; ridx = wave - NSW - 2;
  } else if (wave < NSW + 6) {
    role = R_S; ridx = wave - NSW - 4;
  } else {
    role = R_IDLE; ridx = 0;
  }

  uint32_t cr[NCR];
#pragma unroll
  for (int i = 0; i < NCR; ++i) cr[i] = 0u;

  const int vcol = 16 * ridx + n;  // SCAN: column inside the slice
  if (role == R_SCAN && p.h0 != nullptr) {
    const float* h0 = p.h0 + bi * p.sh0[0] + hi * p.sh0[1] + (v0 + vcol) * p.sh0[3];
#pragma unroll
    for (int r = 0; r < KT; ++r) {
      f32x4 x;
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = h0[(16 * r + 4 * gq + i) * p.sh0[2]];
      cr_setf4(cr, r, x);
    }
  }

  // E: k fragments of its chunk (2 row tiles x KB), then g, beta raw.
  auto e_load = [&](int j) {
    const int t0 = j * C;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
        cr_set4(cr, mt * KB + kb, load_frag(kg, skt, t0 + 16 * mt + n, T, 32 * kb + 8 * gq));
    const int t = t0 + (lane & 31);
    const bool ok = t < T;
    cr[8 * KB] = ok ? load_raw(p.g, g_base + (int64_t)t * p.sg[1], p.g_dtype) : 0u;
    cr[8 * KB + 1] = ok ? load_raw(p.beta, b_base + (int64_t)t * p.sb[1], p.beta_dtype) : 0u;
  };
  // L: q frags [0, 8KB), k frags [8KB, 16KB), v slice, g, beta.
  constexpr int L_V = 16 * KB;          // word offset of the v slice
  constexpr int L_NV = (C * BV / 8 + 63) / 64;  // 16-byte v loads per lane
  constexpr int L_G = L_V + 4 * L_NV;
  static_assert(L_G + 2 <= NCR, "carry too small");
  auto l_load = [&](int j) {
    const int t0 = j * C;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        cr_set4(cr, mt * KB + kb, load_frag(qg, sqt, t0 + 16 * mt + n, T, 32 * kb + 8 * gq));
        cr_set4(cr, 2 * KB + mt * KB + kb,
                load_frag(kg, skt, t0 + 16 * mt + n, T, 32 * kb + 8 * gq));
      }
#pragma unroll
    for (int r = 0; r < L_NV; ++r) {
      const int idx = lane + 64 * r;
      const int t = idx / (BV / 8);
      const int c8 = (idx % (BV / 8)) * 8;
      uint4 x = {0u, 0u, 0u, 0u};
      if (t < C && t0 + t < T) x = *reinterpret_cast<const uint4*>(vg + (int64_t)(t0 + t) * svt + c8);
      cr_set4(cr, L_V / 4 + r, x);
    }
    const int t = t0 + (lane & 31);
    const bool ok = t < T;
    cr[L_G] = ok ? load_raw(p.g, g_base + (int64_t)t * p.sg[1], p.g_dtype) : 0u;
    cr[L_G + 1] = ok ? load_raw(p.beta, b_base + (int64_t)t * p.sb[1], p.beta_dtype) : 0u;
  };

  if (role == R_E && ridx < nch) e_load(ridx);

  for (int it = -8; it < nch; ++it) {
    if (role == R_SCAN) {
      // ------------------------------------------------------------ SCAN
      const int j = it;
      if (j >= 0) {
        const int t0 = j * C;
        const int bs = j % NBIG, ws = j & 1, us = j % NTU;
        const f16* sq = s.q[bs];
        const f16* skt = s.kt[bs];
        const f16* svt = s.vt[bs];
        const f16* sp = s.p[bs];
        const f16* sw = s.w[ws];
        const f16* stu = s.tu[us];
        f16x8 sB[KB];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) sB[kb] = M::from_acc(cr_getf4(cr, 2 * kb), cr_getf4(cr, 2 * kb + 1));
        f32x4 u[2], oq[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          f32x4 acc = M::mma(M::load_pi(stu + (16 * mt + n) * SC, gq),
                             M::load_pi(svt + vcol * SC, gq), f32x4{0.f, 0.f, 0.f, 0.f});
          f32x4 accq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            acc = M::mma(M::load_pi(sw + (16 * mt + n) * SK + 32 * kb, gq), sB[kb], acc);
            accq = M::mma(M::load_pi(sq + (16 * mt + n) * SK + 32 * kb, gq), sB[kb], accq);
          }
          u[mt] = acc;
          oq[mt] = accq;
        }
        f32x4 lo2, hi2;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lo2[i] = u[0][i] * s.ec[bs][4 * gq + i];
          hi2[i] = u[1][i] * s.ec[bs][16 + 4 * gq + i];
        }
        const f16x8 uB = M::from_acc(u[0], u[1]);
        const f16x8 utB = M::from_acc(lo2, hi2);
        // state update first: it is the only thing the next chunk waits for
        const float ebC = s.eb[bs][C - 1];
#pragma unroll
        for (int r = 0; r < KT; ++r) {
          const f32x4 acc = M::mma(M::load_pi(skt + (16 * r + n) * SC, gq), utB, cr_getf4(cr, r) * ebC);
          cr_setf4(cr, r, acc);
        }
        const int64_t o_col = bi * p.so[0] + hi * p.so[2] + v0 + vcol;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const f32x4 acc = M::mma(M::load_pi(sp + (16 * mt + n) * SC, gq), uB, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int t = 16 * mt + 4 * gq + i;
            if (t0 + t < T) {
              const float val = p.scale * (acc[i] + s.eb[bs][t] * oq[mt][i]);
              store_scalar(p.o, o_col + (int64_t)(t0 + t) * p.so[1], p.o_dtype, val);
            }
          }
        }
      }
    } else if (role == R_L) {
      // ------------------------------------------------------------ L
      const int j = it + 2;
      if (j >= 0 && j < nch) {
        const int bs = j % NBIG;
        f16* sq = s.q[bs];
        f16* skt = s.kt[bs];
        f16* svt = s.vt[bs];
        f16* sp = s.p[bs];
        // gates
        const float gt = raw_to_float(cr[L_G], p.g_dtype);
        const float b = scan32(gt, lane);
        const float bC = __shfl(b, C - 1, 64);
        if (lane < C) {
          s.eb[bs][lane] = fexp(b);
          s.ec[bs][lane] = fexp(bC - b);
        }
        // q rows, k^T, v^T
        f16x8 qf[2][KB], kf[2][KB];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            qf[mt][kb] = to_f16x8<TIn>(cr_get4(cr, mt * KB + kb));
            kf[mt][kb] = to_f16x8<TIn>(cr_get4(cr, 2 * KB + mt * KB + kb));
            *reinterpret_cast<f16x8*>(sq + (16 * mt + n) * SK + 32 * kb + 8 * gq) = qf[mt][kb];
#pragma unroll
            for (int e = 0; e < 8; ++e) skt[(32 * kb + 8 * gq + e) * SC + 16 * mt + n] = kf[mt][kb][e];
          }
#pragma unroll
        for (int r = 0; r < L_NV; ++r) {
          const int idx = lane + 64 * r;
          const int t = idx / (BV / 8);
          const int c8 = (idx % (BV / 8)) * 8;
          if (t < C) {
            const f16x8 x = to_f16x8<TIn>(cr_get4(cr, L_V / 4 + r));
#pragma unroll
            for (int e = 0; e < 8; ++e) svt[(c8 + e) * SC + t] = x[e];
          }
        }
        // P = e^{b_t - b_j} (q_t . k_j), j <= t
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) {
            const int jj = 16 * nt + n;
            if (nt > mt) {
#pragma unroll
              for (int i = 0; i < 4; ++i) sp[(16 * mt + 4 * gq + i) * SC + jj] = (f16)0.f;
              continue;
            }
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) acc = M::mma(qf[mt][kb], kf[nt][kb], acc);
            const float bj = __shfl(b, jj, 64);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int t = 16 * mt + 4 * gq + i;
              const float bt = __shfl(b, t, 64);
              sp[t * SC + jj] = (f16)((t >= jj) ? acc[i] * fexp(bt - bj) : 0.f);
            }
          }
        }
      }
      if (j + 1 >= 0 && j + 1 < nch) l_load(j + 1);
    } else if (role == R_WV) {
      // ------------------------------------------------------------ WV
      const int j = it + 1;
      if (j >= 0 && j < nch) {
        const f16* skt = s.kt[j % NBIG];
        const f16* stw = s.tw[j % NTW];
        f16* sw = s.w[j & 1];
#pragma unroll
        for (int mt = 0; mt < KT; ++mt)
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) {
            const f32x4 acc = M::mma(M::load_pi(skt + (16 * mt + n) * SC, gq),
                                     M::load_pi(stw + (16 * nt + n) * SC, gq),
                                     f32x4{0.f, 0.f, 0.f, 0.f});
            M::store4(sw + (16 * nt + n) * SK + 16 * mt + 4 * gq, acc);
          }
      }
    } else if (role == R_E) {
      // ------------------------------------------------------------ E
      const int j = it + 8;
      if (j >= 0 && j < nch && (j & 1) == ridx) {
        const int as = j % NA;
        const float gt = raw_to_float(cr[8 * KB], p.g_dtype);
        const float bt_l = raw_to_float(cr[8 * KB + 1], p.beta_dtype);
        const float b = scan32(gt, lane);
        if (lane < C) {
          s.ab[as][lane] = b;
          s.abeta[as][lane] = bt_l;
        }
        f16x8 kf[2][KB];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) kf[mt][kb] = to_f16x8<TIn>(cr_get4(cr, mt * KB + kb));
        float* sa = s.a[as];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int nt = 0; nt <= mt; ++nt) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) acc = M::mma(kf[mt][kb], kf[nt][kb], acc);
            const int jj = 16 * nt + n;
            const float bj = __shfl(b, jj, 64);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int t = 16 * mt + 4 * gq + i;
              const float bt = __shfl(b, t, 64);
              const float beta_t = __shfl(bt_l, t, 64);
              sa[t * C + jj] = (t > jj) ? acc[i] * fexp(bt - bj) * beta_t : 0.f;
            }
          }
        if (j + 2 < nch) e_load(j + 2);
      }
    } else if (role == R_S) {
      // ------------------------------------------------------------ S
      // pair m' = m + 8 (keeps the arithmetic non-negative)
      const int itp = it + 16;
      int mp = (itp + 4) >> 1;
      if ((mp & 1) != ridx) ++mp;
      const int seg = itp + 6 - 2 * mp;  // 0..3
      const int h = lane >> 5, c = lane & 31;
      const int j = 2 * (mp - 8) + h;
      const bool valid = j >= 0 && j < nch;
      const float* arow = s.a[valid ? j % NA : 0];
      float tc[C];
#pragma unroll
      for (int i = 0; i < C; ++i) tc[i] = __uint_as_float(cr[i]);
      auto rows = [&](auto lo_c, auto hi_c) {
        constexpr int LO = decltype(lo_c)::value, HI = decltype(hi_c)::value;
#pragma unroll
        for (int i = LO; i < HI; ++i) {
          float a0 = (c == i) ? 1.f : 0.f, a1 = 0.f;
#pragma unroll
          for (int j4 = 0; j4 < i; j4 += 4) {
            const f32x4 a4 = *reinterpret_cast<const f32x4*>(arow + i * C + j4);
            float& acc = ((j4 >> 2) & 1) ? a1 : a0;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (j4 + e < i) acc = fmaf(-a4[e], tc[j4 + e], acc);
          }
          tc[i] = a0 + a1;
        }
      };
      if (seg == 0) {
        rows(std::integral_constant<int, 0>{}, std::integral_constant<int, 16>{});
      } else if (seg == 1) {
        rows(std::integral_constant<int, 16>{}, std::integral_constant<int, 23>{});
      } else if (seg == 2) {
        rows(std::integral_constant<int, 23>{}, std::integral_constant<int, 28>{});
      } else {
        rows(std::integral_constant<int, 28>{}, std::integral_constant<int, 32>{});
        if (valid) {
          const int as = j % NA;
          const float ru = s.abeta[as][c];
          const float rw = -ru * fexp(s.ab[as][c]);
          f16* stw = s.tw[j % NTW];
          f16* stu = s.tu[j % NTU];
#pragma unroll
          for (int i = 0; i < C; ++i) {
            stw[i * SC + c] = (f16)(tc[i] * rw);
            stu[i * SC + c] = (f16)(tc[i] * ru);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < C; ++i) cr[i] = __float_as_uint(tc[i]);
    }
    __syncthreads();
  }

  if (role == R_SCAN) {
    float* fs = p.fs + bi * p.sfs[0] + hi * p.sfs[1] + (v0 + vcol) * p.sfs[3];
#pragma unroll
    for (int r = 0; r < KT; ++r) {
      const f32x4 x = cr_getf4(cr, r);
#pragma unroll
      for (int i = 0; i < 4; ++i) fs[(16 * r + 4 * gq + i) * p.sfs[2]] = x[i];
    }
  }
}

template <typename TIn, int K, int BV>
int launch_pipe(const KArgs& a, int grid, hipStream_t stream) {
  static_assert(sizeof(Smem<K, BV>) <= kLdsLimit, "LDS budget");
  hipLaunchKernelGGL((gdn_fwd_pipe_kernel<TIn, K, BV>), dim3(grid), dim3(kThreads8), 0, stream, a);
  return (int)hipGetLastError();
}

}  // namespace pipe

template <typename TIn>
int launch_pipe_k(const KArgs& a, int K, int bv, int grid, hipStream_t s) {
  if (K == 64 && bv == 16) return pipe::launch_pipe<TIn, 64, 16>(a, grid, s);
  if (K == 64 && bv == 32) return pipe::launch_pipe<TIn, 64, 32>(a, grid, s);
  if (K == 128 && bv == 16) return pipe::launch_pipe<TIn, 128, 16>(a, grid, s);
  if (K == 128 && bv == 32) return pipe::launch_pipe<TIn, 128, 32>(a, grid, s);
  return GDN_ERR_UNSUPPORTED;
}

}  // namespace gdn
