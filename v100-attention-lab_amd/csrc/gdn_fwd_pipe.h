// Software-pipelined, wave-specialised GDN forward for fp16/bf16 inputs,
// chunk size C = 32 (the headline configuration).
//
// The phase-by-phase kernel in gdn_fwd_kernel.h spends a chunk's time in a
// serial sequence load -> gates -> K K^T -> substitution -> W -> scan, all
// behind workgroup barriers.  Only u = U + W' S and S <- e^{bC} S + K^T u~
// depend on the previous chunk, so this kernel runs the state-independent
// work of later chunks concurrently with the scan of the current one.  A
// workgroup has 8 waves with fixed roles and exactly one barrier per
// iteration; iteration `it` scans chunk `it` while the other roles work
// ahead:
//
//   role  wave            chunk   work
//   SCAN  0 .. NSW-1      it      u = U + W' S, S <- e^{bC} S + K^T diag(e^{bC-b}) u,
//                                 o = scale (P u + diag(e^b) Q S); then, with
//                                 the new state, Q S and U = Tu V of chunk
//                                 it+1 (so only W' and K^T reads sit between
//                                 the barrier and the state update).
//                                 16 state columns per wave, the state in
//                                 accumulator registers for the whole run.
//   L     NSW             it+2    q rows, K^T and V^T (transposed on the MFMA
//                                 by an identity operand), P = e^{b_t-b_j} Q K^T
//                                 (t >= j), e^b, e^{bC-b} -> "big" slot j % 3
//   WV    NSW+1           it+1    W'^T = K^T Tw^T -> W slot j % 2
//   E0,E1 NSW+2, NSW+3    it+8    gates + A = beta_t e^{b_t-b_j} K K^T (t > j)
//                                 -> A slot j % 6; E_e owns chunks j = e
//                                 (mod 2) and loads them two iterations ahead
//   S0,S1 NSW+4, NSW+5    pairs   forward substitution T = (I+A)^{-1} for two
//                                 chunks at once (lanes 0-31 / 32-63, one
//                                 column per lane, rows of A broadcast from
//                                 LDS), spread over 4 iterations (rows
//                                 [0,16), [16,23), [23,28), [28,32)); writes
//                                 Tw = -T diag(beta e^b) (slot j % 4) and
//                                 Tu = T diag(beta) (slot j % 6)
//
// Pair m = (2m, 2m+1) is solved in iterations 2m-6 .. 2m-3 by S_{m%2}.
// Every slot is written in an earlier iteration than any read of it and is
// not rewritten before its last read (A: written j-8, last read <= j-3;
// Tw: written >= j-4, read j-1; Tu: written >= j-4, read j-1; big: written
// j-2, read j-1 and j; W: written j-1, read j).  Global loads are issued one
// (L) or two (E) iterations before use, so their latency overlaps other
// work; rows past T are clamped and zeroed without branches.
//
// Registers a role carries from one iteration to the next (the state, the
// substitution's column, prefetched tiles) share one array, so the
// kernel's register budget is the largest role's, not the sum.

#pragma once

#include "gdn_fwd_kernel.h"

namespace gdn {

namespace pipe {

constexpr int C = 32;
constexpr int NA = 6, NTW = 4, NTU = 6, NBIG = 3, NWS = 2;

template <int K, int BV>
struct alignas(16) Smem {
  static constexpr int SK = K + 8;   // fp16 row stride of [C][K] tiles
  static constexpr int SC = C + 8;   // fp16 row stride of [*][C] tiles
  static constexpr int NSW = BV / 16;
  // SCAN -> OUT: the fp16 state at a chunk start (B-operand fragments, one
  // 16-byte fragment per lane per 32-row block) and u (one fragment).
  f16x8 so[2][NSW][K / 32][64];
  f16x8 uo[2][NSW][2][64];   // u split as hi + lo (both fp16)
  // OUT -> SCAN: U = Tu V of the next chunk (accumulator tiles).
  f32x4 uc[2][NSW][2][64];
  f16 kt[NBIG][K * SC];
  f16 vt[NBIG][BV * SC];
  f16 p[NBIG][C * SC];
  f16 plo[NBIG][C * SC];  // P - (float)P in fp16: P u is formed as hi*hi + hi*lo + lo*hi
  float bb[NBIG][C];    // in-chunk cumsum b
  float eb[NBIG][C];
  float ec[NBIG][C];
  f16 w[NWS][C * SK];
  f16 tw[NTW][C * SC];
  f16 tu[NTU][C * SC];
  float a[NA][C * C];
  float ab[NA][C];      // in-chunk cumsum b (for Tw's e^{b_j})
  float abeta[NA][C];
};

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

template <typename TIn>
__device__ __forceinline__ f16x8 to_f16x8(const uint4& r) {
  f16 x[8];
  InTraits<TIn>::to_op(r, x);
  return f16x8{x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]};
}

// 8 input elements held as raw 16 bytes in the order they were loaded.
template <typename TIn>
__device__ __forceinline__ f16x8 to_f16x8_pairs(const uint4& r) {
  return to_f16x8<TIn>(r);
}

__device__ __forceinline__ uint4 cr_get4(const uint32_t* cr, int w) {
  return uint4{cr[w], cr[w + 1], cr[w + 2], cr[w + 3]};
}
__device__ __forceinline__ void cr_set4(uint32_t* cr, int w, const uint4& v) {
  cr[w] = v.x;
  cr[w + 1] = v.y;
  cr[w + 2] = v.z;
  cr[w + 3] = v.w;
}
__device__ __forceinline__ f32x4 cr_getf4(const uint32_t* cr, int w) {
  return f32x4{__uint_as_float(cr[w]), __uint_as_float(cr[w + 1]), __uint_as_float(cr[w + 2]),
               __uint_as_float(cr[w + 3])};
}
__device__ __forceinline__ void cr_setf4(uint32_t* cr, int w, const f32x4& v) {
  cr[w] = __float_as_uint(v[0]);
  cr[w + 1] = __float_as_uint(v[1]);
  cr[w + 2] = __float_as_uint(v[2]);
  cr[w + 3] = __float_as_uint(v[3]);
}

// Inclusive prefix sum over lanes 0..31 (and separately 32..63) with DPP:
// shifts by 1, 2, 4, 8 inside each row of 16 lanes (lanes shifted in from
// outside the row read 0), then row_bcast:15 adds the total of rows 0 / 2
// to rows 1 / 3.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_mov0(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, true));
}
__device__ __forceinline__ float scan32(float x, int /*lane*/) {
  x += dpp_mov0<0x111, 0xf>(x);  // row_shr:1
  x += dpp_mov0<0x112, 0xf>(x);  // row_shr:2
  x += dpp_mov0<0x114, 0xf>(x);  // row_shr:4
  x += dpp_mov0<0x118, 0xf>(x);  // row_shr:8
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x142, 0xa, 0xf, false));
  return x;                      // row_bcast:15 into rows 1 and 3
}

// 16 bytes of row min(row, T-1).  Rows past T need no zeroing: their g and
// beta are zeroed where they are used, which makes their rows of A, T, U, W
// and u exactly zero, so whatever finite data they hold contributes nothing
// (and their outputs are not stored).  Not consuming the value here keeps
// the load in flight until the iteration that uses it.
template <typename TIn>
__device__ __forceinline__ uint4 load_row16(const TIn* base, int64_t row_stride, int row, int T,
                                            int col) {
  const int rc = row < T ? row : T - 1;
  return *reinterpret_cast<const uint4*>(base + (int64_t)rc * row_stride + col);
}

// Operand that selects columns [16h, 16h+16) of a 32-wide plain-layout
// block: B[8g + s][n] = (8g + s == 16h + n).  A x I_h is the identity on
// those columns, which turns row fragments into accumulator tiles of the
// transpose (exact: one product with 1.0 per output).
__device__ __forceinline__ f16x8 ident_op(int h, int n, int gq) {
  const int idx = 16 * h + n - 8 * gq;
  f16x8 r;
#pragma unroll
  for (int s = 0; s < 8; ++s) r[s] = (f16)(idx == s ? 1.f : 0.f);
  return r;
}

template <typename TOut>
__device__ __forceinline__ void put(void* o, int64_t off, float x);
template <>
__device__ __forceinline__ void put<float>(void* o, int64_t off, float x) {
  static_cast<float*>(o)[off] = x;
}
template <>
__device__ __forceinline__ void put<f16>(void* o, int64_t off, float x) {
  static_cast<f16*>(o)[off] = (f16)x;
}
template <>
__device__ __forceinline__ void put<bf16_t>(void* o, int64_t off, float x) {
  static_cast<uint16_t*>(o)[off] = float_to_bf16_bits(x);
}

// Output rows 16 mt + 4 gq + i of one 16-column block.
template <typename TOut>
__device__ __forceinline__ void store_o(void* o, int64_t col_off, int64_t row_stride, int t0, int T,
                                        int gq, const f32x4 (&val)[2]) {
  if (t0 + C <= T) {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        put<TOut>(o, col_off + (int64_t)(t0 + 16 * mt + 4 * gq + i) * row_stride, val[mt][i]);
  } else {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = t0 + 16 * mt + 4 * gq + i;
        if (t < T) put<TOut>(o, col_off + (int64_t)t * row_stride, val[mt][i]);
      }
  }
}

// Rows [LO, HI) of the forward substitution for the column this lane owns:
// T[i][c] = [i == c] - sum_{j<i} A[i][j] T[j][c].  Row i+1 of A is read
// from LDS while row i is computed.
template <int LO, int HI>
__device__ __forceinline__ void solve_rows(const float* arow, int c, float (&tc)[C]) {
  constexpr int NQ = (HI - 1 + 3) / 4;  // float4s of the longest row
  f32x4 cur[NQ > 0 ? NQ : 1];
#pragma unroll
  for (int q4 = 0; q4 < (LO + 3) / 4; ++q4)
    cur[q4] = *reinterpret_cast<const f32x4*>(arow + LO * C + 4 * q4);
#pragma unroll
  for (int i = LO; i < HI; ++i) {
    f32x4 nxt[NQ > 0 ? NQ : 1];
    if (i + 1 < HI) {
#pragma unroll
      for (int q4 = 0; q4 < (i + 1 + 3) / 4; ++q4)
        nxt[q4] = *reinterpret_cast<const f32x4*>(arow + (i + 1) * C + 4 * q4);
    }
    float a0 = (c == i) ? 1.f : 0.f, a1 = 0.f;
#pragma unroll
    for (int q4 = 0; q4 < (i + 3) / 4; ++q4) {
      float& acc = (q4 & 1) ? a1 : a0;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (4 * q4 + e < i) acc = fmaf(-cur[q4][e], tc[4 * q4 + e], acc);
    }
    tc[i] = a0 + a1;
    if (i + 1 < HI) {
#pragma unroll
      for (int q4 = 0; q4 < (i + 1 + 3) / 4; ++q4) cur[q4] = nxt[q4];
    }
  }
}

// ---------------------------------------------------------------------------

template <int BV>
constexpr int pipe_waves() {
  return 7 + BV / 16;
}

template <typename TIn, int K, int BV>
__global__ __launch_bounds__(64 * pipe_waves<BV>()) void gdn_fwd_pipe_kernel(const KArgs p) {
  using M = Mma<f16>;
  using S = Smem<K, BV>;
  constexpr int SK = S::SK, SC = S::SC;
  constexpr int NSW = BV / 16;
  constexpr int KB = K / 32, KT = K / 16;
  static_assert(NSW >= 1 && NSW <= 2, "BV must be 16 or 32");
  static_assert(K == 64 || K == 128, "K must be 64 or 128");

  __shared__ S s;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};

  // Raw g, beta of row min(t0 + (lane & 31), T-1); rows past T are zeroed
  // where the values are used (gate_at).
  auto load_gb = [&](uint32_t* dst, int j) {
    const int t = j * C + (lane & 31);
    const int tc = t < T ? t : T - 1;
    dst[0] = load_raw(p.g, g_base + (int64_t)tc * p.sg[1], p.g_dtype);
    dst[1] = load_raw(p.beta, b_base + (int64_t)tc * p.sb[1], p.beta_dtype);
  };
  auto gate_at = [&](int j, uint32_t raw, int dtype) {
    const float x = raw_to_float(raw, dtype);
    return j * C + (lane & 31) < T ? x : 0.f;
  };
  // Row fragments (2 row tiles x KB blocks, plain layout) of a [*, K] input.
  auto load_rows = [&](uint32_t* dst, const TIn* base, int64_t stride, int j) {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
        cr_set4(dst, 4 * (mt * KB + kb),
                load_row16(base, stride, j * C + 16 * mt + n, T, 32 * kb + 8 * gq));
  };

  // Roles, in wave order: SCAN x NSW, OUT, L, E0, WV, S0, S1, E1 (waves map
  // to SIMDs round-robin, which pairs each heavy role with a lighter one).
  enum { R_SCAN, R_OUT, R_L, R_E, R_WV, R_S, R_IDLE };
  int role = R_IDLE, ridx = 0;
  {
    const int w = wave - NSW;
    if (wave < NSW) { role = R_SCAN; ridx = wave; }
    else if (w == 0) role = R_OUT;
    else if (w == 1) role = R_L;
    else if (w == 2) { role = R_E; ridx = 0; }
    else if (w == 3) role = R_WV;
    else if (w == 4) { role = R_S; ridx = 0; }
    else if (w == 5) { role = R_S; ridx = 1; }
    else if (w == 6) { role = R_E; ridx = 1; }
  }

  // Each role runs its own copy of the iteration loop, so registers that one
  // role keeps live across iterations cost nothing in the others; every
  // wave executes exactly one barrier per iteration.
  if (role == R_SCAN) {
    // ================================================================ SCAN
    // chunk it: u = U + W' S, S <- e^{bC} S + K^T diag(e^{bC-b}) u; hands
    // u and the new fp16 state to OUT.
    const int cb = ridx;
    const int vcol = 16 * cb + n;
    f32x4 st[KT];
#pragma unroll
    for (int r = 0; r < KT; ++r) st[r] = z4;
    if (p.h0 != nullptr) {
      const float* h0 = p.h0 + bi * p.sh0[0] + hi * p.sh0[1] + (v0 + vcol) * p.sh0[3];
#pragma unroll
      for (int r = 0; r < KT; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) st[r][i] = h0[(16 * r + 4 * gq + i) * p.sh0[2]];
    }
    f16x8 sB[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      sB[kb] = M::from_acc(st[2 * kb], st[2 * kb + 1]);
      s.so[0][cb][kb][lane] = sB[kb];
    }
    for (int it = -8; it < nch; ++it) {
      const int j = it;
      if (j >= 0) {
        const int bs = j % NBIG;
        const f16* sk = s.kt[bs];
        const f16* sw = s.w[j & 1];
        f16x8 wA[2][KB], kA[KT];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) wA[mt][kb] = M::load_pi(sw + (16 * mt + n) * SK + 32 * kb, gq);
#pragma unroll
        for (int r = 0; r < KT; ++r) kA[r] = M::load_pi(sk + (16 * r + n) * SC, gq);
        f32x4 u[2] = {s.uc[j & 1][cb][0][lane], s.uc[j & 1][cb][1][lane]};
        const f32x4 ec_lo = *reinterpret_cast<const f32x4*>(&s.ec[bs][4 * gq]);
        const f32x4 ec_hi = *reinterpret_cast<const f32x4*>(&s.ec[bs][16 + 4 * gq]);
        const float ebC = s.eb[bs][C - 1];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) u[mt] = M::mma(wA[mt][kb], sB[kb], u[mt]);
        const f16x8 utB = M::from_acc(u[0] * ec_lo, u[1] * ec_hi);
#pragma unroll
        for (int r = 0; r < KT; ++r) st[r] = M::mma(kA[r], utB, st[r] * ebC);
        {
          const f16x8 uh = M::from_acc(u[0], u[1]);
          s.uo[j & 1][cb][0][lane] = uh;
          s.uo[j & 1][cb][1][lane] = split_lo(u[0], u[1], uh);
        }
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          sB[kb] = M::from_acc(st[2 * kb], st[2 * kb + 1]);
          s.so[(j + 1) & 1][cb][kb][lane] = sB[kb];
        }
      }
      __syncthreads();
    }
    float* fs = p.fs + bi * p.sfs[0] + hi * p.sfs[1] + (v0 + vcol) * p.sfs[3];
#pragma unroll
    for (int r = 0; r < KT; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) fs[(16 * r + 4 * gq + i) * p.sfs[2]] = st[r][i];
  } else if (role == R_OUT) {
    // ================================================================ OUT
    // chunk it: Q S (q from global, S from SCAN); chunk it-1:
    // o = scale (P u + diag(e^b) Q S) -> o; chunk it+1: U = Tu V -> SCAN.
    // q fragments in the pi layout: two 8-byte pieces per 32-block.
    uint2 qr[2][KB][2];
    f16x8 pA[2], pL[2];
    f32x4 ebv[2], oq[NSW][2];
    auto load_q = [&](int j) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int row = j * C + 16 * mt + n;
        const int rc = row < T ? row : T - 1;
        const TIn* qrow = qg + (int64_t)rc * sqt;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          qr[mt][kb][0] = *reinterpret_cast<const uint2*>(qrow + 32 * kb + 4 * gq);
          qr[mt][kb][1] = *reinterpret_cast<const uint2*>(qrow + 32 * kb + 16 + 4 * gq);
        }
      }
    };
    auto store_chunk = [&](int j) {
#pragma unroll
      for (int c2 = 0; c2 < NSW; ++c2) {
        const f16x8 uh = s.uo[j & 1][c2][0][lane];
        const f16x8 ul = s.uo[j & 1][c2][1][lane];
        f32x4 ov[2];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          f32x4 pu = M::mma(pA[mt], ul, z4);
          pu = M::mma(pL[mt], uh, pu);
          pu = M::mma(pA[mt], uh, pu);
          ov[mt] = (pu + ebv[mt] * oq[c2][mt]) * p.scale;
        }
        const int64_t o_col = bi * p.so[0] + hi * p.so[2] + v0 + 16 * c2 + n;
        if (p.o_dtype == GDN_DTYPE_F16)
          store_o<f16>(p.o, o_col, p.so[1], j * C, T, gq, ov);
        else if (p.o_dtype == GDN_DTYPE_BF16)
          store_o<bf16_t>(p.o, o_col, p.so[1], j * C, T, gq, ov);
        else
          store_o<float>(p.o, o_col, p.so[1], j * C, T, gq, ov);
      }
    };
#pragma unroll
    for (int c2 = 0; c2 < NSW; ++c2) oq[c2][0] = oq[c2][1] = z4;
    ebv[0] = ebv[1] = z4;
    pA[0] = pA[1] = pL[0] = pL[1] = f16x8{};
    for (int it = -8; it < nch; ++it) {
      const int j = it;
      if (j >= 1) store_chunk(j - 1);  // o of chunk j-1 (u_{j-1} written in it-1)
      if (j >= 0) {
        // Q S of chunk j with S_j (written by SCAN in it-1)
        f16x8 qA[2][KB];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            const uint4 r4 = {qr[mt][kb][0].x, qr[mt][kb][0].y, qr[mt][kb][1].x, qr[mt][kb][1].y};
            qA[mt][kb] = to_f16x8_pairs<TIn>(r4);
          }
#pragma unroll
        for (int c2 = 0; c2 < NSW; ++c2)
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) {
            f32x4 acc = z4;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) acc = M::mma(qA[mt][kb], s.so[j & 1][c2][kb][lane], acc);
            oq[c2][mt] = acc;
          }
        // P and e^b of chunk j for its output in the next iteration
        const int bs = j % NBIG;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          pA[mt] = M::load_pi(s.p[bs] + (16 * mt + n) * SC, gq);
          pL[mt] = M::load_pi(s.plo[bs] + (16 * mt + n) * SC, gq);
        }
        ebv[0] = *reinterpret_cast<const f32x4*>(&s.eb[bs][4 * gq]);
        ebv[1] = *reinterpret_cast<const f32x4*>(&s.eb[bs][16 + 4 * gq]);
      }
      const int jn = it + 1;
      if (jn >= 0 && jn < nch) {
        const int bs = jn % NBIG;
        const f16* stu = s.tu[jn % NTU];
        const f16x8 tu0 = M::load_pi(stu + n * SC, gq);
        const f16x8 tu1 = M::load_pi(stu + (16 + n) * SC, gq);
#pragma unroll
        for (int c2 = 0; c2 < NSW; ++c2) {
          const f16x8 vB = M::load_pi(s.vt[bs] + (16 * c2 + n) * SC, gq);
          s.uc[jn & 1][c2][0][lane] = M::mma(tu0, vB, z4);
          s.uc[jn & 1][c2][1][lane] = M::mma(tu1, vB, z4);
        }
        load_q(jn);
      }
      __syncthreads();
    }
    if (nch > 0) store_chunk(nch - 1);
  } else if (role == R_L) {
    // ================================================================ L
    // chunk it+2: gates and P = e^{b_t-b_j} Q K^T (t >= j)
    constexpr int QW = 0, KW = 8 * KB, GW = 16 * KB;
    uint32_t cr[16 * KB + 2];
    for (int it = -8; it < nch; ++it) {
      const int j = it + 2;
      if (j >= 0 && j < nch) {
        const int bs = j % NBIG;
        f16* sp = s.p[bs];
        f16* spl = s.plo[bs];
        const float b = scan32(gate_at(j, cr[GW], p.g_dtype), lane);
        const float bC = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(b), C - 1));
        if (lane < C) {
          s.bb[bs][lane] = b;
          s.eb[bs][lane] = fexp(b);
          s.ec[bs][lane] = fexp(bC - b);
        }
        f16x8 qf[2][KB], kf[2][KB];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            qf[mt][kb] = to_f16x8<TIn>(cr_get4(cr, QW + 4 * (mt * KB + kb)));
            kf[mt][kb] = to_f16x8<TIn>(cr_get4(cr, KW + 4 * (mt * KB + kb)));
          }
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) {
            const int jj = 16 * nt + n;
            if (nt > mt) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                sp[(16 * mt + 4 * gq + i) * SC + jj] = (f16)0.f;
                spl[(16 * mt + 4 * gq + i) * SC + jj] = (f16)0.f;
              }
              continue;
            }
            f32x4 acc = z4;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) acc = M::mma(qf[mt][kb], kf[nt][kb], acc);
            const float bj = s.bb[bs][jj];
            const f32x4 bt4 = *reinterpret_cast<const f32x4*>(&s.bb[bs][16 * mt + 4 * gq]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int t = 16 * mt + 4 * gq + i;
              // mask folded into the exponent: 2^-inf = 0
              const float x = t >= jj ? bt4[i] - bj : -__builtin_inff();
              const float pv = acc[i] * fexp(x);
              const f16 ph = (f16)pv;
              sp[t * SC + jj] = ph;
              spl[t * SC + jj] = (f16)(pv - (float)ph);
            }
          }
        }
      }
      if (j + 1 >= 0 && j + 1 < nch) {
        load_rows(cr + QW, qg, sqt, j + 1);
        load_rows(cr + KW, kg, skt, j + 1);
        load_gb(cr + GW, j + 1);
      }
      __syncthreads();
    }
  } else if (role == R_WV) {
    // ================================================================ WV
    // chunk it+2: K^T and V^T transposed on the MFMA (X I_h = columns
    // [16h, 16h+16) of X as accumulator tiles of X^T); chunk it+1:
    // W'^T = K^T Tw^T.
    constexpr int KW = 0, VW = 8 * KB;
    uint32_t cr[8 * KB + 8];
    const f16x8 id0 = ident_op(0, n, gq), id1 = ident_op(1, n, gq);
    for (int it = -8; it < nch; ++it) {
      const int jw = it + 1;
      if (jw >= 0 && jw < nch) {
        const f16* sk = s.kt[jw % NBIG];
        const f16* stw = s.tw[jw % NTW];
        f16* sw = s.w[jw & 1];
        f16x8 kA[KT], tB[2];
#pragma unroll
        for (int mt = 0; mt < KT; ++mt) kA[mt] = M::load_pi(sk + (16 * mt + n) * SC, gq);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) tB[nt] = M::load_pi(stw + (16 * nt + n) * SC, gq);
#pragma unroll
        for (int mt = 0; mt < KT; ++mt)
#pragma unroll
          for (int nt = 0; nt < 2; ++nt)
            M::store4(sw + (16 * nt + n) * SK + 16 * mt + 4 * gq, M::mma(kA[mt], tB[nt], z4));
      }
      const int j = it + 2;
      if (j >= 0 && j < nch) {
        const int bs = j % NBIG;
        f16* sk = s.kt[bs];
        f16* sv = s.vt[bs];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
          for (int c = 0; c < KT; ++c) {
            const f16x8 kf = to_f16x8<TIn>(cr_get4(cr, KW + 4 * (mt * KB + (c >> 1))));
            M::store4(sk + (16 * c + n) * SC + 16 * mt + 4 * gq, M::mma(kf, (c & 1) ? id1 : id0, z4));
          }
          const f16x8 vf = to_f16x8<TIn>(cr_get4(cr, VW + 4 * mt));
#pragma unroll
          for (int c = 0; c < BV / 16; ++c)
            M::store4(sv + (16 * c + n) * SC + 16 * mt + 4 * gq, M::mma(vf, (c & 1) ? id1 : id0, z4));
        }
      }
      if (j + 1 >= 0 && j + 1 < nch) {
        load_rows(cr + KW, kg, skt, j + 1);
        // v slice: lane (n, gq) reads columns [8 gq, +8); lanes with
        // 8 gq >= BV read a duplicate the transpose never selects
        const int cv = 8 * gq < BV ? 8 * gq : BV - 8;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
          cr_set4(cr, VW + 4 * mt, load_row16(vg, svt, (j + 1) * C + 16 * mt + n, T, cv));
      }
      __syncthreads();
    }
  } else if (role == R_E) {
    // ================================================================ E
    // chunk it+8 (E_e owns chunks = e mod 2): gates, A = beta_t e^{b_t-b_j} K K^T
    const int e = ridx;
    constexpr int KW = 0, GW = 8 * KB;
    uint32_t cr[8 * KB + 2];
    auto e_load = [&](int j) {
      load_rows(cr + KW, kg, skt, j);
      load_gb(cr + GW, j);
    };
    if (e < nch) e_load(e);
    for (int it = -8; it < nch; ++it) {
      const int j = it + 8;
      if (j >= 0 && j < nch && (j & 1) == e) {
        const int as = j % NA;
        const float b = scan32(gate_at(j, cr[GW], p.g_dtype), lane);
        const float bet = gate_at(j, cr[GW + 1], p.beta_dtype);
        if (lane < C) {
          s.ab[as][lane] = b;
          s.abeta[as][lane] = bet;
        }
        f16x8 kf[2][KB];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) kf[mt][kb] = to_f16x8<TIn>(cr_get4(cr, KW + 4 * (mt * KB + kb)));
        float* sa = s.a[as];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int nt = 0; nt <= mt; ++nt) {
            f32x4 acc = z4;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) acc = M::mma(kf[mt][kb], kf[nt][kb], acc);
            const int jj = 16 * nt + n;
            const float bj = s.ab[as][jj];
            const f32x4 bt4 = *reinterpret_cast<const f32x4*>(&s.ab[as][16 * mt + 4 * gq]);
            const f32x4 be4 = *reinterpret_cast<const f32x4*>(&s.abeta[as][16 * mt + 4 * gq]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int t = 16 * mt + 4 * gq + i;
              const float x = t > jj ? bt4[i] - bj : -__builtin_inff();
              sa[t * C + jj] = acc[i] * fexp(x) * be4[i];
            }
          }
        if (j + 2 < nch) e_load(j + 2);
      }
      __syncthreads();
    }
  } else if (role == R_S) {
    // ================================================================ S
    // pair m = (2m, 2m+1) in iterations 2m-6 .. 2m-3; m' = m + 8 keeps the
    // arithmetic non-negative
    const int sidx = ridx;
    const int h = lane >> 5, c = lane & 31;
    float tc[C];
#pragma unroll
    for (int i = 0; i < C; ++i) tc[i] = 0.f;
    for (int it = -8; it < nch; ++it) {
      const int itp = it + 16;
      int mp = (itp + 4) >> 1;
      if ((mp & 1) != sidx) ++mp;
      const int seg = itp + 6 - 2 * mp;  // 0..3
      const int j = 2 * (mp - 8) + h;
      const bool valid = j >= 0 && j < nch;
      const float* arow = s.a[valid ? j % NA : 0];
      if (seg == 0) {
        solve_rows<0, 16>(arow, c, tc);
      } else if (seg == 1) {
        solve_rows<16, 23>(arow, c, tc);
      } else if (seg == 2) {
        solve_rows<23, 28>(arow, c, tc);
      } else {
        solve_rows<28, 32>(arow, c, tc);
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
      __syncthreads();
    }
  } else {
    for (int it = -8; it < nch; ++it) __syncthreads();
  }
}

template <typename TIn, int K, int BV>
int launch_pipe(const KArgs& a, int grid, hipStream_t stream) {
  static_assert(sizeof(Smem<K, BV>) <= kLdsLimit, "LDS budget");
  hipLaunchKernelGGL((gdn_fwd_pipe_kernel<TIn, K, BV>), dim3(grid), dim3(64 * pipe_waves<BV>()), 0,
                     stream, a);
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
