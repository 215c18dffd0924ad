// The forward for 64-row chunks, as two launches (fp16, bf16 and fp32
// inputs; K in {32, 64, 128}; fp32 arithmetic on v_mfma_f32_16x16x4_f32).
//
// Per chunk (C = 64 rows, b = in-chunk cumsum of g, gam = e^b, D_j =
// e^{bC - b_j}, M[t][j] = e^{b_t - b_j} for j <= t), as in gdn_ref.py:48-99:
//   A = tril_-1(beta_t M K K^T),  T = (I + A)^-1,  W = T diag(beta gam) K,
//   u = T diag(beta) V - W S,
//   o = scale (P u + diag(gam) Q S),  P = M o (Q K^T),
//   S' = gam_C S + K^T diag(D) u.
// Only u, o and S' involve the carried state S.  With 64-row chunks the
// state-independent half (the K K^T and Q K^T products, the 64 x 64
// substitution, W) is the larger one, and it runs first, for every chunk at
// once:
//   1. prep_kernel, one workgroup per (chunk, head): gates, T (two 32 x 32
//      diagonal solves, one lane per column, then the off-diagonal block
//      T21 = -T22 A21 T11 on the matrix cores), W and P, written to a
//      per-chunk record in the caller's workspace;
//   2. scan_kernel, one workgroup per (sequence, head, 16-column V slice):
//      walks the chunks with S resident in LDS (O(B H K V) state: no chunk
//      state is written), loading the next chunk's record and rows while the
//      current one computes.  Waves 0-3 compute u (16 rows each), then the
//      state update; waves 4-7 compute Q S for the same rows, then o.
// Packed sequences (cu_seqlens) number their chunk slots floor(t0 / C) + i
// onwards, as in the backward.

#include "gdn_tiles_f32.h"

namespace gdn {
namespace c64 {

using namespace tiles;

constexpr int C = 64;
constexpr int BV = 16;
constexpr int NT = 512;   // threads of both kernels (8 waves)
constexpr int UNR = 8;    // contraction steps unrolled in the products
// LDS rows padded to a multiple of 4 floats: 16-byte stores when staging,
// at most 2-way bank conflicts on the operand reads
constexpr int PAD = 4;

struct FArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  const float* h0;
  void* o;
  float* fs;
  float* rec;
  int64_t sq[3], sk[3], sv[3], sg[3], sb[3], so[3];
  int64_t sh0[4], sfs[4];
  int B, T, H, V, nv, nchmax, units;
  float scale;
  int g_dtype, beta_dtype, o_dtype;
  const int64_t* cu;
  int xcd_remap;
};

// Per-(slot, head) record, in floats: T and P as [C][C], W as [C][K], then
// gam and D as [C] each and gam_C (first of a [C] row).
template <int K>
struct Rec {
  static constexpr int T = 0, PM = C * C, W = 2 * C * C;
  static constexpr int G = W + C * K;
  static constexpr int SIZE = G + 3 * C;
};
inline int64_t rec_size(int K) { return 2 * C * C + (int64_t)C * K + 3 * C; }

// The record for 16-bit inputs, in the same bytes: P, W and T diag(beta) as
// fp16 hi + lo pairs (x = hi + lo to about 2^-22 relative; offsets in
// halves), then the gates as floats (offset GF in floats).
template <int K>
struct Rec16 {
  static constexpr int PH = 0, PL = C * C, WH = 2 * C * C, WL = 2 * C * C + C * K;
  static constexpr int TH = 2 * C * C + 2 * C * K, TL = 3 * C * C + 2 * C * K;
  static constexpr int NH = 4 * C * C + 2 * C * K;
  static constexpr int GF = NH / 2;
};
static_assert(Rec16<128>::GF + 3 * C == Rec<128>::SIZE && Rec16<32>::GF + 3 * C == Rec<32>::SIZE,
              "the two records take the same bytes");

// x as an fp16 pair hi + lo.
__device__ __forceinline__ void split_f16(float x, f16& hi, f16& lo) {
  x = pin(x);
  hi = (f16)x;
  lo = (f16)(x - (float)hi);
}

// ---------------------------------------------------------------------------
// 1. prep
// ---------------------------------------------------------------------------

template <int K>
struct alignas(16) PSmem {
  float q[C][K + PAD], k[C][K + PAD];
  float a[C][C + PAD];   // K K^T, then A
  float qk[C][C + PAD];  // Q K^T, then A21 T11
  float t[C][C + PAD];
  float gl[C], bt[C], b[C], gam[C], D[C];
  float gC;
};

template <typename TIn, int K>
__global__ __launch_bounds__(NT) void prep_kernel(const FArgs p) {
  using R = Rec<K>;
  __shared__ PSmem<K> s;
  const int tid = threadIdx.x;
  const int64_t slot = blockIdx.x / p.H;
  const int hi = blockIdx.x % p.H;
  RowSpan rs;
  int c;
  if (!slot_chunk<C>(p, slot, rs, c)) return;
  const int t0 = c * C, nval = min(C, rs.T - t0);
  float* const rec = p.rec + (slot * p.H + hi) * (int64_t)R::SIZE;

  {
    RowLoad<TIn, C, K, NT> lq, lk;
    lq.load(tid, static_cast<const TIn*>(p.q) + head_base(rs, hi, p.sq) + t0 * p.sq[1], p.sq[1], nval);
    lk.load(tid, static_cast<const TIn*>(p.k) + head_base(rs, hi, p.sk) + t0 * p.sk[1], p.sk[1], nval);
    float gv = 0.f, bv = 0.f;
    if (tid < nval) {
      gv = load_scalar(p.g, head_base(rs, hi, p.sg) + (int64_t)(t0 + tid) * p.sg[1], p.g_dtype);
      bv = load_scalar(p.beta, head_base(rs, hi, p.sb) + (int64_t)(t0 + tid) * p.sb[1], p.beta_dtype);
    }
    lq.store(tid, s.q);
    lk.store(tid, s.k);
    if (tid < C) {
      s.gl[tid] = gv;
      s.bt[tid] = bv;
    }
  }
  __syncthreads();
  if (tid < C) {
    // sequential cumsum in each lane (the association order of a plain
    // running sum)
    float bt = 0.f, bc = 0.f;
    for (int j = 0; j < C; ++j) {
      bc += s.gl[j];
      if (j == tid) bt = bc;
    }
    s.b[tid] = bt;
    s.gam[tid] = expf(bt);
    s.D[tid] = expf(bc - bt);
    if (tid == C - 1) s.gC = expf(bc);
  }
  if constexpr (std::is_same<TIn, float>::value) {
    mmx<NT, C, C, UNR>(tid, [&](int m, int n, float x) { s.a[m][n] = x; },
                       seg<K>([&](int m, int kk) { return s.k[m][kk]; }, [&](int kk, int n) { return s.k[n][kk]; }));
    mmx<NT, C, C, UNR>(tid, [&](int m, int n, float x) { s.qk[m][n] = x; },
                       seg<K>([&](int m, int kk) { return s.q[m][kk]; }, [&](int kk, int n) { return s.k[n][kk]; }));
  } else {
    // 16-bit inputs are exact in fp16 (bf16 values within the fp16 range,
    // as in the fused kernels): K K^T and Q K^T on v_mfma_f32_16x16x32_f16,
    // exact products with fp32 accumulation.  Lane (r, kq) supplies 8
    // consecutive k of row r; 2 x 16 tiles over the 8 waves.
    const int lane = tid & 63, r = lane & 15, kq = lane >> 4;
    auto frag8 = [&](const float* row) {
      const f32x4 lo = *reinterpret_cast<const f32x4*>(row), hi = *reinterpret_cast<const f32x4*>(row + 4);
      return f16x8{(f16)lo[0], (f16)lo[1], (f16)lo[2], (f16)lo[3], (f16)hi[0], (f16)hi[1], (f16)hi[2], (f16)hi[3]};
    };
    for (int job = tid >> 6; job < 2 * (C / 16) * (C / 16); job += NT / 64) {
      const int mat = job / ((C / 16) * (C / 16)), mt = (job / (C / 16)) % (C / 16), nt = job % (C / 16);
      const float* arow = (mat ? &s.q[0][0] : &s.k[0][0]) + (16 * mt + r) * (K + PAD) + 8 * kq;
      const float* brow = &s.k[0][0] + (16 * nt + r) * (K + PAD) + 8 * kq;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < K / 32; ++kb)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag8(arow + 32 * kb), frag8(brow + 32 * kb), acc, 0, 0, 0);
      float(*dst)[C + PAD] = mat ? s.qk : s.a;
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[16 * mt + 4 * kq + i][16 * nt + r] = acc[i];
    }
  }
  __syncthreads();
  constexpr bool kF32 = std::is_same<TIn, float>::value;
  using R16 = Rec16<K>;
  f16* const rh = reinterpret_cast<f16*>(rec);
  for (int e = tid; e < C * C; e += NT) {
    const int t = e / C, j = e % C;
    const float mv = j <= t ? expf(s.b[t] - s.b[j]) : 0.f;
    if constexpr (kF32) {
      rec[R::PM + e] = mv * s.qk[t][j];
    } else {
      split_f16(mv * s.qk[t][j], rh[R16::PH + e], rh[R16::PL + e]);
    }
    s.a[t][j] = j < t ? s.bt[t] * mv * s.a[t][j] : 0.f;
  }
  if (tid < C) {
    float* const gr = kF32 ? rec + R::G : rec + R16::GF;
    gr[tid] = s.gam[tid];
    gr[C + tid] = s.D[tid];
    gr[2 * C + tid] = tid == 0 ? s.gC : 0.f;
  }
  __syncthreads();
  // T11 = (I + A11)^-1 (lanes 0-31 of wave 0) and T22 = (I + A22)^-1 (lanes
  // 0-31 of wave 1): one column per lane, the column in registers
  if ((tid & 63) < 32 && tid < 128) {
    const int o = tid < 64 ? 0 : 32, cc = tid & 31;
    float col[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      float x = (i == cc) ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j) x = __builtin_fmaf(-s.a[o + i][o + j], col[j], x);
      col[i] = x;
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      s.t[o + i][o + cc] = col[i];
      s.t[o + i][32 - o + cc] = 0.f;  // T12 = 0 (and T21 overwritten below)
    }
  }
  __syncthreads();
  // X = A21 T11 -> qk
  mmx<NT, 32, 32, UNR>(tid, [&](int m, int n, float x) { s.qk[m][n] = x; },
                  seg<32>([&](int m, int kk) { return s.a[32 + m][kk]; }, [&](int kk, int n) { return s.t[kk][n]; }));
  __syncthreads();
  // T21 = -T22 X
  mmx<NT, 32, 32, UNR>(tid, [&](int m, int n, float x) { s.t[32 + m][n] = -x; },
                  seg<32>([&](int m, int kk) { return s.t[32 + m][32 + kk]; },
                          [&](int kk, int n) { return s.qk[kk][n]; }));
  __syncthreads();
  if constexpr (kF32) {
    for (int e = tid; e < C * C; e += NT) rec[R::T + e] = s.t[e / C][e % C];
  } else {
    // T diag(beta), the operand of U = T diag(beta) V
    for (int e = tid; e < C * C; e += NT)
      split_f16(s.t[e / C][e % C] * s.bt[e % C], rh[R16::TH + e], rh[R16::TL + e]);
  }
  // W = T diag(beta gam) K
  mmx<NT, C, K, UNR>(tid,
                     [&](int m, int n, float x) {
                       if constexpr (kF32) rec[R::W + m * K + n] = x;
                       else split_f16(x, rh[R16::WH + m * K + n], rh[R16::WL + m * K + n]);
                     },
                     seg<C>([&](int m, int kk) { return s.t[m][kk]; },
                            [&](int kk, int n) { return s.bt[kk] * s.gam[kk] * s.k[kk][n]; }));
}

// ---------------------------------------------------------------------------
// 2. scan
// ---------------------------------------------------------------------------

template <int K>
struct alignas(16) SSmem {
  float S[K][BV + 1];
  float t[C][C + PAD], pm[C][C + PAD];
  float w[C][K + PAD], q[C][K + PAD], k[C][K + PAD];
  float v[C][BV + PAD], u[C][BV + 1];
  float bt[C], gam[C], D[C];
  float gC;
};

// Next chunk's record and rows, in registers.  Scalars are kept as raw bits
// and converted when stored: a conversion right after the load would make
// the wave wait for every load issued before it.
template <typename TIn, int K>
struct Next {
  using R = Rec<K>;
  RowLoad<float, C, C, NT> lt, lp;
  RowLoad<float, C, K, NT> lw;
  RowLoad<TIn, C, K, NT> lq, lk;
  RowLoad<TIn, C, BV, NT> lv;
  uint32_t bv;
  float gm, dv, gc;
  __device__ __forceinline__ void load(const FArgs& p, int tid, int64_t ri, const TIn* qg, const TIn* kg,
                                       const TIn* vg, int64_t bb, int t0, int nval) {
    const float* const rec = p.rec + ri * R::SIZE;
    lt.load(tid, rec + R::T, C, C);
    lp.load(tid, rec + R::PM, C, C);
    lw.load(tid, rec + R::W, K, C);
    lq.load(tid, qg + (int64_t)t0 * p.sq[1], p.sq[1], nval);
    lk.load(tid, kg + (int64_t)t0 * p.sk[1], p.sk[1], nval);
    lv.load(tid, vg + (int64_t)t0 * p.sv[1], p.sv[1], nval);
    bv = tid < nval ? load_bits(p.beta, bb + (int64_t)(t0 + tid) * p.sb[1], p.beta_dtype) : 0u;
    gm = tid < C ? rec[R::G + tid] : 0.f;
    dv = tid < C ? rec[R::G + C + tid] : 0.f;
    gc = tid == 0 ? rec[R::G + 2 * C] : 0.f;
  }
  __device__ __forceinline__ void store(SSmem<K>& s, int tid, int beta_dtype) const {
    lt.store(tid, s.t);
    lp.store(tid, s.pm);
    lw.store(tid, s.w);
    lq.store(tid, s.q);
    lk.store(tid, s.k);
    lv.store(tid, s.v);
    if (tid < C) {
      s.bt[tid] = bits_to_float(bv, beta_dtype);
      s.gam[tid] = gm;
      s.D[tid] = dv;
    }
    if (tid == 0) s.gC = gc;
  }
};

template <typename TIn, int K>
__global__ __launch_bounds__(NT) void scan_kernel(const FArgs p) {
  __shared__ SSmem<K> s;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, kq = lane >> 4;
  int unit = blockIdx.x;
  if (p.xcd_remap) unit = (blockIdx.x & 7) * (p.units >> 3) + (blockIdx.x >> 3);
  const int vs = unit % p.nv;
  const int bh = unit / p.nv;
  const int bi = bh / p.H;
  const int hi = bh % p.H;
  const int v0 = vs * BV;
  const RowSpan rs = row_span(p.cu, p.T, bi);
  const int64_t slot0 = p.cu ? rs.t0 / C + bi : (int64_t)bi * p.nchmax;
  const int nch = (rs.T + C - 1) / C;
  const float scale = p.scale;
  const TIn* const qg = static_cast<const TIn*>(p.q) + head_base(rs, hi, p.sq);
  const TIn* const kg = static_cast<const TIn*>(p.k) + head_base(rs, hi, p.sk);
  const TIn* const vg = static_cast<const TIn*>(p.v) + head_base(rs, hi, p.sv) + v0;
  const int64_t bb = head_base(rs, hi, p.sb);
  const int64_t ob = head_base(rs, hi, p.so) + v0;

  for (int e = tid; e < K * BV; e += NT) {
    const int kk = e / BV, c2 = e % BV;
    s.S[kk][c2] = p.h0 ? p.h0[bi * p.sh0[0] + hi * p.sh0[1] + kk * p.sh0[2] + (v0 + c2) * p.sh0[3]] : 0.f;
  }
  Next<TIn, K> nx;
  if (nch > 0) {
    nx.load(p, tid, slot0 * p.H + hi, qg, kg, vg, bb, 0, min(C, rs.T));
    nx.store(s, tid, p.beta_dtype);
  }
  __syncthreads();
  // waves 0-3: u rows 16 w .., then the state update; waves 4-7: Q S rows
  // 16 (w - 4) .., then o of those rows
  const int um0 = 16 * (wave & 3);
  constexpr int NST = (K / 16 + 3) / 4;  // state tiles per wave: rows 16 (w + 4 j)
  for (int c = 0; c < nch; ++c) {
    const int t0 = c * C, nval = min(C, rs.T - t0);
    if (c + 1 < nch)
      nx.load(p, tid, (slot0 + c + 1) * p.H + hi, qg, kg, vg, bb, t0 + C, min(C, rs.T - t0 - C));
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (wave < 4) {
      // u = T diag(beta) V - W S
#pragma unroll UNR
      for (int k0 = 0; k0 < C; k0 += 4)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(s.t[um0 + r][k0 + kq], s.bt[k0 + kq] * s.v[k0 + kq][r], acc,
                                                   0, 0, 0);
#pragma unroll UNR
      for (int k0 = 0; k0 < K; k0 += 4)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(-s.w[um0 + r][k0 + kq], s.S[k0 + kq][r], acc, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) s.u[um0 + 4 * kq + i][r] = acc[i];
    } else {
      // Q S, kept for o
#pragma unroll UNR
      for (int k0 = 0; k0 < K; k0 += 4)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(s.q[um0 + r][k0 + kq], s.S[k0 + kq][r], acc, 0, 0, 0);
    }
    __syncthreads();
    if (wave < 4) {
      // S <- gam_C S + K^T diag(D) u
      f32x4 as[NST];
#pragma unroll
      for (int j = 0; j < NST; ++j) as[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll UNR
      for (int k0 = 0; k0 < C; k0 += 4) {
        const float ub = s.u[k0 + kq][r], d = s.D[k0 + kq];
#pragma unroll
        for (int j = 0; j < NST; ++j)
          if (wave + 4 * j < K / 16)
            as[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(s.k[k0 + kq][16 * (wave + 4 * j) + r] * d, ub, as[j],
                                                         0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < NST; ++j)
        if (wave + 4 * j < K / 16) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = 16 * (wave + 4 * j) + 4 * kq + i;
            s.S[m][r] = s.gC * s.S[m][r] + as[j][i];
          }
        }
    } else {
      // o = scale (P u + diag(gam) Q S)
      f32x4 ao = {0.f, 0.f, 0.f, 0.f};
#pragma unroll UNR
      for (int k0 = 0; k0 < C; k0 += 4)
        ao = __builtin_amdgcn_mfma_f32_16x16x4f32(s.pm[um0 + r][k0 + kq], s.u[k0 + kq][r], ao, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = um0 + 4 * kq + i;
        if (row < nval)
          store_scalar(p.o, ob + (int64_t)(t0 + row) * p.so[1] + r, p.o_dtype,
                       scale * (ao[i] + s.gam[row] * acc[i]));
      }
    }
    __syncthreads();
    if (c + 1 < nch) {
      nx.store(s, tid, p.beta_dtype);
      __syncthreads();
    }
  }
  for (int e = tid; e < K * BV; e += NT) {
    const int kk = e / BV, c2 = e % BV;
    p.fs[bi * p.sfs[0] + hi * p.sfs[1] + kk * p.sfs[2] + (v0 + c2) * p.sfs[3]] = s.S[kk][c2];
  }
}

// ---------------------------------------------------------------------------
// 2b. scan for 16-bit inputs: fp16 MFMA on hi + lo operand pairs
// ---------------------------------------------------------------------------
//
// v_mfma_f32_16x16x32_f16 contracts 32 at once: lane (r, kq) supplies row r
// of A and row r of B^T, 8 consecutive contraction indices 8 kq .. from
// each 32-block, so every operand is stored with the contraction index
// contiguous (K^T, V^T, S^T and u^T transposed).  q, k and v are exact in
// fp16; every fp32 operand is an fp16 pair hi + lo, and a product of two
// fp32 values is hi*hi + hi*lo + lo*hi (to about 2^-22 relative).  The
// fp32 state S lives in the accumulators of waves 0-3 (rows 16 (w + 4 j)
// of K); its hi / lo copies in LDS feed W S and Q S.

constexpr int HP = 8;  // LDS row padding in halves (rows stay 16-byte aligned)

template <int K>
struct alignas(16) S16mem {
  f16 sh[BV][K + HP], sl[BV][K + HP];  // S^T
  f16 wh[C][K + HP], wl[C][K + HP];
  f16 q[C][K + HP];
  f16 kt[K][C + HP];                   // K^T
  f16 th[C][C + HP], tl[C][C + HP];    // T diag(beta)
  f16 ph[C][C + HP], pl[C][C + HP];    // P
  f16 vt[BV][C + HP];                  // V^T of the slice
  f16 uh[BV][C + HP], ul[BV][C + HP];  // u^T
  f16 dh[BV][C + HP], dl[BV][C + HP];  // (diag(D) u)^T
  float gam[C], D[C];
  float gC;
};

__device__ __forceinline__ f16x8 frag8(const f16* p) { return *reinterpret_cast<const f16x8*>(p); }

// ROWS x COLS halves, rows `ld` halves apart in global memory -> LDS rows of
// LD halves, 16 bytes per lane.
template <int ROWS, int COLS>
struct HalfRows {
  static constexpr int RV = COLS / 8, NV = ROWS * RV, N = (NV + NT - 1) / NT;
  u32x4 r[N];
  __device__ __forceinline__ void load(int tid, const f16* src, int64_t ld) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT;
      if (e < NV) r[i] = *reinterpret_cast<const u32x4*>(src + (e / RV) * ld + (e % RV) * 8);
    }
  }
  template <int LD>
  __device__ __forceinline__ void store(int tid, f16 (*dst)[LD]) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT;
      if (e < NV) *reinterpret_cast<u32x4*>(&dst[e / RV][(e % RV) * 8]) = r[i];
    }
  }
};

// ROWS x COLS block of a 16-bit input (rows >= nvalid read as zero) in
// 8-element vectors, handed out row-fastest (vector e: row e % ROWS) so that
// the transposed LDS stores of a wave hit consecutive halves.
template <typename TIn, int ROWS, int COLS>
struct InRows {
  static constexpr int RV = COLS / 8, NV = ROWS * RV, N = (NV + NT - 1) / NT;
  uint4 r[N];
  __device__ __forceinline__ void load(int tid, const TIn* src, int64_t ld, int nvalid, bool transposed) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT;
      const int t = transposed ? e % ROWS : e / RV, c = transposed ? e / ROWS : e % RV;
      r[i] = uint4{0u, 0u, 0u, 0u};
      if (e < NV && t < nvalid) r[i] = *reinterpret_cast<const uint4*>(src + t * ld + 8 * c);
    }
  }
  // dst[t][8c + j] (row-major) or dst[8c + j][t] (transposed), as fp16
  template <int LD>
  __device__ __forceinline__ void store(int tid, f16 (*dst)[LD], bool transposed) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int e = tid + i * NT;
      if (e >= NV) continue;
      f16 x[8];
      InTraits<TIn>::to_op(r[i], x);
      if (transposed) {
        const int t = e % ROWS, c = e / ROWS;
#pragma unroll
        for (int j = 0; j < 8; ++j) dst[8 * c + j][t] = x[j];
      } else {
        *reinterpret_cast<f16x8*>(&dst[e / RV][8 * (e % RV)]) =
            f16x8{x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]};
      }
    }
  }
};

// Next chunk's record and rows, in registers.
template <typename TIn, int K>
struct Next16 {
  using R = Rec16<K>;
  HalfRows<C, C> ph, pl, th, tl;
  HalfRows<C, K> wh, wl;
  InRows<TIn, C, K> q, k;
  InRows<TIn, C, BV> v;
  float gm, dv, gc;
  __device__ __forceinline__ void load(const FArgs& p, int tid, int64_t ri, const TIn* qg, const TIn* kg,
                                       const TIn* vg, int t0, int nval) {
    const float* const rec = p.rec + ri * (int64_t)Rec<K>::SIZE;
    const f16* const rh = reinterpret_cast<const f16*>(rec);
    ph.load(tid, rh + R::PH, C);
    pl.load(tid, rh + R::PL, C);
    th.load(tid, rh + R::TH, C);
    tl.load(tid, rh + R::TL, C);
    wh.load(tid, rh + R::WH, K);
    wl.load(tid, rh + R::WL, K);
    q.load(tid, qg + (int64_t)t0 * p.sq[1], p.sq[1], nval, false);
    k.load(tid, kg + (int64_t)t0 * p.sk[1], p.sk[1], nval, true);
    v.load(tid, vg + (int64_t)t0 * p.sv[1], p.sv[1], nval, true);
    gm = tid < C ? rec[R::GF + tid] : 0.f;
    dv = tid < C ? rec[R::GF + C + tid] : 0.f;
    gc = tid == 0 ? rec[R::GF + 2 * C] : 0.f;
  }
  __device__ __forceinline__ void store(S16mem<K>& s, int tid) const {
    ph.store(tid, s.ph);
    pl.store(tid, s.pl);
    th.store(tid, s.th);
    tl.store(tid, s.tl);
    wh.store(tid, s.wh);
    wl.store(tid, s.wl);
    q.store(tid, s.q, false);
    k.store(tid, s.kt, true);
    v.store(tid, s.vt, true);
    if (tid < C) {
      s.gam[tid] = gm;
      s.D[tid] = dv;
    }
    if (tid == 0) s.gC = gc;
  }
};

template <typename TIn, int K>
__global__ __launch_bounds__(NT) void scan16_kernel(const FArgs p) {
  __shared__ S16mem<K> s;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, kq = lane >> 4;
  int unit = blockIdx.x;
  if (p.xcd_remap) unit = (blockIdx.x & 7) * (p.units >> 3) + (blockIdx.x >> 3);
  const int vs = unit % p.nv;
  const int bh = unit / p.nv;
  const int bi = bh / p.H;
  const int hi = bh % p.H;
  const int v0 = vs * BV;
  const RowSpan rs = row_span(p.cu, p.T, bi);
  const int64_t slot0 = p.cu ? rs.t0 / C + bi : (int64_t)bi * p.nchmax;
  const int nch = (rs.T + C - 1) / C;
  const float scale = p.scale;
  const TIn* const qg = static_cast<const TIn*>(p.q) + head_base(rs, hi, p.sq);
  const TIn* const kg = static_cast<const TIn*>(p.k) + head_base(rs, hi, p.sk);
  const TIn* const vg = static_cast<const TIn*>(p.v) + head_base(rs, hi, p.sv) + v0;
  const int64_t ob = head_base(rs, hi, p.so) + v0;

  // waves 0-3: the state rows 16 (w + 4 j) of K (accumulator layout: rows
  // 4 kq + i, column r), u rows 16 w; waves 4-7: Q S and o rows 16 (w - 4)
  constexpr int NST = (K / 16 + 3) / 4;
  const bool upper = wave < 4;
  const int um0 = 16 * (wave & 3);
  f32x4 st[NST];
  // S^T hi / lo for the products with S
  auto put_state = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NST; ++j) {
      const int m0 = 16 * (wave + 4 * j);
      if (m0 < K) {
        f16 h[4], l[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) split_f16(st[j][i], h[i], l[i]);
        *reinterpret_cast<f16x4*>(&s.sh[r][m0 + 4 * kq]) = f16x4{h[0], h[1], h[2], h[3]};
        *reinterpret_cast<f16x4*>(&s.sl[r][m0 + 4 * kq]) = f16x4{l[0], l[1], l[2], l[3]};
      }
    }
  };
  if (upper) {
#pragma unroll
    for (int j = 0; j < NST; ++j) {
      const int m0 = 16 * (wave + 4 * j);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st[j][i] = (p.h0 && m0 < K)
                       ? p.h0[bi * p.sh0[0] + hi * p.sh0[1] + (m0 + 4 * kq + i) * p.sh0[2] + (v0 + r) * p.sh0[3]]
                       : 0.f;
    }
    put_state();
  }
  Next16<TIn, K> nx;
  if (nch > 0) {
    nx.load(p, tid, slot0 * p.H + hi, qg, kg, vg, 0, min(C, rs.T));
    nx.store(s, tid);
  }
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    const int t0 = c * C, nval = min(C, rs.T - t0);
    if (c + 1 < nch) nx.load(p, tid, (slot0 + c + 1) * p.H + hi, qg, kg, vg, t0 + C, min(C, rs.T - t0 - C));
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (upper) {
      // u = T diag(beta) V - W S for rows um0 ..
      f32x4 aw = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jb = 0; jb < C; jb += 32) {
        const f16x8 b = frag8(&s.vt[r][jb + 8 * kq]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag8(&s.th[um0 + r][jb + 8 * kq]), b, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag8(&s.tl[um0 + r][jb + 8 * kq]), b, acc, 0, 0, 0);
      }
#pragma unroll
      for (int kb = 0; kb < K; kb += 32) {
        const f16x8 wh = frag8(&s.wh[um0 + r][kb + 8 * kq]), sh = frag8(&s.sh[r][kb + 8 * kq]);
        aw = __builtin_amdgcn_mfma_f32_16x16x32_f16(wh, sh, aw, 0, 0, 0);
        aw = __builtin_amdgcn_mfma_f32_16x16x32_f16(wh, frag8(&s.sl[r][kb + 8 * kq]), aw, 0, 0, 0);
        aw = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag8(&s.wl[um0 + r][kb + 8 * kq]), sh, aw, 0, 0, 0);
      }
      // u^T and (diag(D) u)^T as fp16 pairs: lane holds u rows um0 + 4 kq + i, column r
      f16 uh[4], ul[4], dh[4], dl[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float u = acc[i] - aw[i];
        split_f16(u, uh[i], ul[i]);
        split_f16(s.D[um0 + 4 * kq + i] * u, dh[i], dl[i]);
      }
      *reinterpret_cast<f16x4*>(&s.uh[r][um0 + 4 * kq]) = f16x4{uh[0], uh[1], uh[2], uh[3]};
      *reinterpret_cast<f16x4*>(&s.ul[r][um0 + 4 * kq]) = f16x4{ul[0], ul[1], ul[2], ul[3]};
      *reinterpret_cast<f16x4*>(&s.dh[r][um0 + 4 * kq]) = f16x4{dh[0], dh[1], dh[2], dh[3]};
      *reinterpret_cast<f16x4*>(&s.dl[r][um0 + 4 * kq]) = f16x4{dl[0], dl[1], dl[2], dl[3]};
    } else {
      // Q S for rows um0 .. (q exact in fp16)
#pragma unroll
      for (int kb = 0; kb < K; kb += 32) {
        const f16x8 a = frag8(&s.q[um0 + r][kb + 8 * kq]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, frag8(&s.sh[r][kb + 8 * kq]), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, frag8(&s.sl[r][kb + 8 * kq]), acc, 0, 0, 0);
      }
    }
    __syncthreads();
    if (upper) {
      // S <- gam_C S + K^T diag(D) u (k exact in fp16)
#pragma unroll
      for (int j = 0; j < NST; ++j) {
        const int m0 = 16 * (wave + 4 * j);
        if (m0 < K) {
          f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int tb = 0; tb < C; tb += 32) {
            const f16x8 kt = frag8(&s.kt[m0 + r][tb + 8 * kq]);
            a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kt, frag8(&s.dh[r][tb + 8 * kq]), a, 0, 0, 0);
            a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kt, frag8(&s.dl[r][tb + 8 * kq]), a, 0, 0, 0);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) st[j][i] = s.gC * st[j][i] + a[i];
        }
      }
      put_state();
    } else {
      // o = scale (P u + diag(gam) Q S)
      f32x4 ao = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jb = 0; jb < C; jb += 32) {
        const f16x8 ph = frag8(&s.ph[um0 + r][jb + 8 * kq]), uh = frag8(&s.uh[r][jb + 8 * kq]);
        ao = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, uh, ao, 0, 0, 0);
        ao = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, frag8(&s.ul[r][jb + 8 * kq]), ao, 0, 0, 0);
        ao = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag8(&s.pl[um0 + r][jb + 8 * kq]), uh, ao, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = um0 + 4 * kq + i;
        if (row < nval)
          store_scalar(p.o, ob + (int64_t)(t0 + row) * p.so[1] + r, p.o_dtype,
                       scale * (ao[i] + s.gam[row] * acc[i]));
      }
    }
    __syncthreads();
    if (c + 1 < nch) {
      nx.store(s, tid);
      __syncthreads();
    }
  }
  if (upper) {
#pragma unroll
    for (int j = 0; j < NST; ++j) {
      const int m0 = 16 * (wave + 4 * j);
      if (m0 < K) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          p.fs[bi * p.sfs[0] + hi * p.sfs[1] + (m0 + 4 * kq + i) * p.sfs[2] + (v0 + r) * p.sfs[3]] = st[j][i];
      }
    }
  }
}

template <typename TIn, int K>
int launch_k(const FArgs& a, int64_t nrec, hipStream_t s) {
  if (nrec > 0) hipLaunchKernelGGL((prep_kernel<TIn, K>), dim3((unsigned)nrec), dim3(NT), 0, s, a);
  if constexpr (std::is_same<TIn, float>::value)
    hipLaunchKernelGGL((scan_kernel<TIn, K>), dim3(a.units), dim3(NT), 0, s, a);
  else
    hipLaunchKernelGGL((scan16_kernel<TIn, K>), dim3(a.units), dim3(NT), 0, s, a);
  return (int)hipGetLastError();
}

template <typename TIn>
int launch_t(const FArgs& a, int K, int64_t nrec, hipStream_t s) {
  switch (K) {
    case 32: return launch_k<TIn, 32>(a, nrec, s);
    case 64: return launch_k<TIn, 64>(a, nrec, s);
    case 128: return launch_k<TIn, 128>(a, nrec, s);
    default: return GDN_ERR_UNSUPPORTED;
  }
}

inline int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

}  // namespace c64

// Chunk slots x heads x record size, in bytes.
int64_t c64_workspace_size(int B, int T, int H, int K, int n_seq) {
  const int64_t nch = (T + c64::C - 1) / c64::C;
  const int64_t nslot = n_seq > 0 ? nch + n_seq : (int64_t)B * nch;
  return c64::align256(nslot * H * c64::rec_size(K) * 4);
}

bool c64_supported(int K, int C, int V) { return C == c64::C && (K == 32 || K == 64 || K == 128) && V % 16 == 0; }

// Enqueue the two launches (arguments checked by the caller).
int c64_launch(const GdnFwdParams& P, hipStream_t stream) {
  const int n_seq = P.cu_seqlens ? P.B : 0;
  c64::FArgs a = {};
  a.q = P.q; a.k = P.k; a.v = P.v; a.g = P.g; a.beta = P.beta; a.h0 = P.h0;
  a.o = P.o; a.fs = P.final_state;
  a.rec = static_cast<float*>(P.workspace);
  for (int d = 0; d < 3; ++d) {
    a.sq[d] = P.q_stride[d]; a.sk[d] = P.k_stride[d]; a.sv[d] = P.v_stride[d];
    a.sg[d] = P.g_stride[d]; a.sb[d] = P.beta_stride[d]; a.so[d] = P.o_stride[d];
  }
  for (int d = 0; d < 4; ++d) { a.sh0[d] = P.h0_stride[d]; a.sfs[d] = P.fs_stride[d]; }
  a.B = P.B; a.T = P.T; a.H = P.H; a.V = P.V; a.nv = P.V / c64::BV;
  a.nchmax = (P.T + c64::C - 1) / c64::C;
  const int64_t units = (int64_t)P.B * P.H * a.nv;
  a.units = (int)units;
  a.scale = P.scale;
  a.g_dtype = P.g_dtype; a.beta_dtype = P.beta_dtype; a.o_dtype = P.o_dtype;
  a.cu = P.cu_seqlens;
  a.xcd_remap = (units % 8 == 0) ? 1 : 0;
  const int64_t nslot = n_seq > 0 ? a.nchmax + n_seq : (int64_t)P.B * a.nchmax;
  const int64_t nrec = P.T > 0 ? nslot * P.H : 0;
  if (nrec > 0x7fffffffLL) return GDN_ERR_BAD_SHAPE;
  switch (P.qkv_dtype) {
    case GDN_DTYPE_F16: return c64::launch_t<f16>(a, P.K, nrec, stream);
    case GDN_DTYPE_BF16: return c64::launch_t<bf16_t>(a, P.K, nrec, stream);
    default: return c64::launch_t<float>(a, P.K, nrec, stream);
  }
}

}  // namespace gdn
