// The forward for 64-row chunks, as two launches (fp16, bf16 and fp32
// inputs; K in {32, 64, 128}).
//
// Per chunk (C = 64 rows, b = in-chunk cumsum of g, gam = e^b, D_j =
// e^{bC - b_j}, M[t][j] = e^{b_t - b_j} for j <= t), as in gdn_ref.py:48-99:
//   A = tril_-1(beta_t M K K^T),  T = (I + A)^-1,  W = T diag(beta gam) K,
//   u = T diag(beta) V - W S = T diag(beta) (V - diag(gam) K S),
//   o = scale (P u + diag(gam) Q S),  P = M o (Q K^T),
//   S' = gam_C S + K^T diag(D) u.
// Only u, o and S' involve the carried state S.  The 64 x 64 substitution
// for T is the long serial step and does not depend on S; it runs first,
// for every chunk at once:
//   1. prep, one workgroup per (chunk, head): gates and T on the VALU, as
//      block forward substitution (the two 32 x 32 diagonal blocks by
//      substitution at once, one lane per column, then the lower-left block
//      T21 = -T22 A21 T11 as dot products over LDS rows), written to a
//      per-chunk record in the caller's workspace;
//   2. scan, one workgroup per (sequence, head, 16-column V slice): walks
//      the chunks with S on chip (no chunk state is written), loading the
//      next chunk's record and rows while the current one computes.
// fp32 inputs (prep_kernel, scan_kernel: fp32 MFMA) keep T, P and W in the
// record.  16-bit inputs (prep16_kernel, scan16_kernel: fp16 MFMA on hi + lo
// pairs) keep T diag(beta), P and the gates there; the scan forms K S, u and
// o from the q, k, v rows it loads anyway, and reads 67 KB per chunk and V
// slice (K = 128; 98 KB with W in the record).
// The records of a segment of L chunks per (sequence, head) live in the
// caller's workspace, [sequence][head][L]: a sequence of more than L chunks
// runs as several (prep, scan) pairs, the state passing from one segment to
// the next through final_state (in fp32, so the result does not depend on
// L).  The workspace is bounded by B * H * L records, independent of T.

#include "gdn_tiles_f16.h"

namespace gdn {
namespace c64 {

using namespace tiles;
using namespace tiles16;

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
  int B, T, H, V, nv, nchmax, units;  // B: sequences (units of row_span)
  int c0, L;   // this segment: chunks [c0, c0 + L) of every sequence
  int first;   // initial state from h0 (or zero) rather than final_state
  float scale;
  int g_dtype, beta_dtype, o_dtype;
  const int64_t* cu;
  int xcd_remap;
  int o_vec;  // o rows take 4-element vector stores (base and strides aligned)
};

// Record workgroup -> (sequence rows, chunk, record index).  The workgroups
// of a segment enumerate (j, sequence, head), head fastest; record
// ((sequence * H) + head) * L + j holds chunk c0 + j.  False past the end of
// the sequence.
__device__ __forceinline__ bool seg_chunk(const FArgs& p, int64_t blk, RowSpan& rs, int& c, int64_t& ri) {
  const int hi = (int)(blk % p.H);
  const int64_t rest = blk / p.H;
  const int bi = (int)(rest % p.B);
  const int j = (int)(rest / p.B);
  rs = row_span(p.cu, p.T, bi);
  c = p.c0 + j;
  ri = ((int64_t)bi * p.H + hi) * p.L + j;
  return (int64_t)c * C < rs.T;
}

// Per-(slot, head) record for fp32 inputs, in floats: T and P as [C][C], W
// as [C][K], then gam and D as [C] each and gam_C (first of a [C] row).
template <int K>
struct Rec {
  static constexpr int T = 0, PM = C * C, W = 2 * C * C;
  static constexpr int G = W + C * K;
  static constexpr int SIZE = G + 3 * C;
};
// The record for 16-bit inputs: T diag(beta) and P as fp16 pairs hi + lo
// (x = hi + lo to about 2^-22 relative; offsets TH, TL, PH, PL in halves),
// then gam, D and b as [C] floats each and gam_C (first of a [C] row;
// offset GF in floats).
struct Rec16 {
  static constexpr int TH = 0, TL = C * C, PH = 2 * C * C, PL = 3 * C * C;
  static constexpr int GF = 2 * C * C;
  static constexpr int SIZE = GF + 4 * C;
};
// floats per record (fp32 or 16-bit inputs)
constexpr int64_t rec_floats(int K, bool half) { return half ? Rec16::SIZE : 2 * C * C + (int64_t)C * K + 3 * C; }
static_assert(Rec<128>::SIZE == rec_floats(128, false) && Rec<32>::SIZE == rec_floats(32, false), "record sizes");

// ---------------------------------------------------------------------------
// 1. prep
// ---------------------------------------------------------------------------

// In-chunk gates from g (gl), in lanes 0 .. C-1: b as a plain running sum
// (the association order of a sequential cumsum), gam = e^b, D = e^{b_C - b}
// and gam_C.
__device__ __forceinline__ void chunk_gates(int tid, const float* gl, float* b, float* gam, float* D, float& gC) {
  if (tid < C) {
    float bt = 0.f, bc = 0.f;
    for (int j = 0; j < C; ++j) {
      bc += gl[j];
      if (j == tid) bt = bc;
    }
    b[tid] = bt;
    gam[tid] = expf(bt);
    D[tid] = expf(bc - bt);
    if (tid == C - 1) gC = expf(bc);
  }
}

// T = (I + A)^-1 for a strictly lower 64 x 64 A, given as at = A^T (a
// barrier passed since it was written), all on the VALU, as the block form
// of forward substitution:
//   * T11 = (I + A11)^-1 and T22 = (I + A22)^-1 by forward substitution at
//     the same time, lanes 0-31 of waves 0 and 1, one column per lane held
//     in registers, the rows of A broadcast from LDS (right-looking: once
//     v[j] is final it is subtracted from every row below; row i still sums
//     its terms in the order j = 0, 1, .., but the dependent chain is 32
//     steps long, not 496);
//   * the second block row, (I + A22) T21 = -A21 T11: X = A21 T11 (x: 32 x
//     32 scratch), then T21 = -T22 X, as VALU dot products over LDS rows
//     (every thread two entries of each).
// T12 = 0.  Ends with a barrier.
template <int XLD>
__device__ __forceinline__ void solve_t(int tid, float (*at)[C + PAD], float (*t)[C + PAD], float (*x)[XLD]) {
  if ((tid & 63) < 32 && tid < 128) {
    const int o = tid < 64 ? 0 : 32, cc = tid & 31;
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = (i == cc) ? 1.f : 0.f;
#pragma unroll
    for (int j = 0; j < 32; ++j)
#pragma unroll
      for (int i = j + 1; i < 32; ++i) v[i] = __builtin_fmaf(-at[o + j][o + i], v[j], v[i]);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      t[o + i][o + cc] = v[i];
      t[o + i][32 - o + cc] = 0.f;  // T12 = 0 (and T21, overwritten below)
    }
  }
  __syncthreads();
  // X = A21 T11 (T11's zeros above its diagonal are exact)
  for (int e = tid; e < 32 * 32; e += NT) {
    const int m = e / 32, n = e % 32;
    float acc = 0.f;
#pragma unroll 8
    for (int kk = 0; kk < 32; ++kk) acc = __builtin_fmaf(at[kk][32 + m], t[kk][n], acc);
    x[m][n] = acc;
  }
  __syncthreads();
  // T21 = -T22 X
  for (int e = tid; e < 32 * 32; e += NT) {
    const int m = e / 32, n = e % 32;
    float acc = 0.f;
#pragma unroll 8
    for (int kk = 0; kk < 32; ++kk) acc = __builtin_fmaf(t[32 + m][32 + kk], x[kk][n], acc);
    t[32 + m][n] = -acc;
  }
  __syncthreads();
}

template <int K>
struct alignas(16) PSmem {
  float q[C][K + PAD], k[C][K + PAD];
  float a[C][C + PAD];   // (K K^T)^T, then A^T
  float qk[C][C + PAD];  // Q K^T, then A21 T11
  float t[C][C + PAD];
  float gl[C], bt[C], b[C], gam[C], D[C];
  float gC;
};

// fp32 inputs: record T, P, W and the gates.
template <int K>
__global__ __launch_bounds__(NT) void prep_kernel(const FArgs p) {
  using R = Rec<K>;
  __shared__ PSmem<K> s;
  const int tid = threadIdx.x;
  RowSpan rs;
  int c;
  int64_t ri;
  if (!seg_chunk(p, blockIdx.x, rs, c, ri)) return;
  const int t0 = c * C, nval = min(C, rs.T - t0);
  const int hi = blockIdx.x % p.H;
  float* const rec = p.rec + ri * (int64_t)R::SIZE;

  {
    RowLoad<float, C, K, NT> lq, lk;
    lq.load(tid, static_cast<const float*>(p.q) + head_base(rs, hi, p.sq) + t0 * p.sq[1], p.sq[1], nval);
    lk.load(tid, static_cast<const float*>(p.k) + head_base(rs, hi, p.sk) + t0 * p.sk[1], p.sk[1], nval);
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
  chunk_gates(tid, s.gl, s.b, s.gam, s.D, s.gC);
  mmx<NT, C, C, UNR>(tid, [&](int m, int n, float x) { s.a[n][m] = x; },
                     seg<K>([&](int m, int kk) { return s.k[m][kk]; }, [&](int kk, int n) { return s.k[n][kk]; }));
  mmx<NT, C, C, UNR>(tid, [&](int m, int n, float x) { s.qk[m][n] = x; },
                     seg<K>([&](int m, int kk) { return s.q[m][kk]; }, [&](int kk, int n) { return s.k[n][kk]; }));
  __syncthreads();
  for (int e = tid; e < C * C; e += NT) {
    const int t = e / C, j = e % C;
    const float mv = j <= t ? expf(s.b[t] - s.b[j]) : 0.f;
    rec[R::PM + e] = mv * s.qk[t][j];
    s.a[j][t] = j < t ? s.bt[t] * mv * s.a[j][t] : 0.f;  // A^T
  }
  if (tid < C) {
    rec[R::G + tid] = s.gam[tid];
    rec[R::G + C + tid] = s.D[tid];
    rec[R::G + 2 * C + tid] = tid == 0 ? s.gC : 0.f;
  }
  __syncthreads();
  solve_t<C + PAD>(tid, s.a, s.t, s.qk);
  for (int e = tid; e < C * C; e += NT) rec[R::T + e] = s.t[e / C][e % C];
  // W = T diag(beta gam) K
  mmx<NT, C, K, UNR>(tid, [&](int m, int n, float x) { rec[R::W + m * K + n] = x; },
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
  // this segment's chunks [c0, c0 + nloc) and their records
  const int nloc = max(0, min(p.L, (rs.T + C - 1) / C - p.c0));
  if (nloc == 0 && !p.first) return;  // state unchanged
  const int64_t rb = ((int64_t)bi * p.H + hi) * p.L;
  const float scale = p.scale;
  const TIn* const qg = static_cast<const TIn*>(p.q) + head_base(rs, hi, p.sq);
  const TIn* const kg = static_cast<const TIn*>(p.k) + head_base(rs, hi, p.sk);
  const TIn* const vg = static_cast<const TIn*>(p.v) + head_base(rs, hi, p.sv) + v0;
  const int64_t bb = head_base(rs, hi, p.sb);
  const int64_t ob = head_base(rs, hi, p.so) + v0;

  for (int e = tid; e < K * BV; e += NT) {
    const int kk = e / BV, c2 = e % BV;
    const int64_t off = kk * p.sfs[2] + (v0 + c2) * p.sfs[3];
    s.S[kk][c2] = !p.first ? p.fs[bi * p.sfs[0] + hi * p.sfs[1] + off]
                  : p.h0   ? p.h0[bi * p.sh0[0] + hi * p.sh0[1] + kk * p.sh0[2] + (v0 + c2) * p.sh0[3]]
                           : 0.f;
  }
  Next<TIn, K> nx;
  if (nloc > 0) {
    const int t0 = p.c0 * C;
    nx.load(p, tid, rb, qg, kg, vg, bb, t0, min(C, rs.T - t0));
    nx.store(s, tid, p.beta_dtype);
  }
  __syncthreads();
  // waves 0-3: u rows 16 w .., then the state update; waves 4-7: Q S rows
  // 16 (w - 4) .., then o of those rows
  const int um0 = 16 * (wave & 3);
  constexpr int NST = (K / 16 + 3) / 4;  // state tiles per wave: rows 16 (w + 4 j)
  for (int j = 0; j < nloc; ++j) {
    const int t0 = (p.c0 + j) * C, nval = min(C, rs.T - t0);
    if (j + 1 < nloc) nx.load(p, tid, rb + j + 1, qg, kg, vg, bb, t0 + C, min(C, rs.T - t0 - C));
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
    if (j + 1 < nloc) {
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
// 3. 16-bit inputs: fp16 MFMA on hi + lo operand pairs
// ---------------------------------------------------------------------------
//
// v_mfma_f32_16x16x32_f16: lane (r, kq) (r = lane % 16, kq = lane / 16)
// supplies row r of A and row r of B^T, 8 consecutive contraction indices
// 8 kq .. from each 32-block, so every operand is stored with the
// contraction index contiguous; the accumulator holds rows 4 kq + i,
// column r.  q, k and v are exact in fp16 (bf16 values within the fp16
// range, as in the fused kernels); every fp32 operand is an fp16 pair
// hi + lo, and a product of two fp32 values is hi*hi + hi*lo + lo*hi (to
// about 2^-22 relative).

// o[base + i * rs] = v[i] for the i < lim of 4 consecutive rows.
template <typename TOut>
__device__ __forceinline__ void store_o4(void* o, int64_t base, int64_t rs, int lim, const float (&v)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (i < lim) {
      if constexpr (std::is_same<TOut, f16>::value) static_cast<f16*>(o)[base + i * rs] = (f16)v[i];
      else if constexpr (std::is_same<TOut, bf16_t>::value) static_cast<uint16_t*>(o)[base + i * rs] = float_to_bf16_bits(v[i]);
      else static_cast<float*>(o)[base + i * rs] = v[i];
    }
  }
}

// 4 consecutive elements of o at o + off (aligned for the vector store).
template <typename TOut>
__device__ __forceinline__ void store_o_vec4(void* o, int64_t off, const f32x4& v) {
  if constexpr (std::is_same<TOut, f16>::value) {
    *reinterpret_cast<f16x4*>(static_cast<f16*>(o) + off) = f16x4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
  } else if constexpr (std::is_same<TOut, bf16_t>::value) {
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(o) + off) =
        uint2{float_to_bf16_bits(v[0]) | ((uint32_t)float_to_bf16_bits(v[1]) << 16),
              float_to_bf16_bits(v[2]) | ((uint32_t)float_to_bf16_bits(v[3]) << 16)};
  } else {
    *reinterpret_cast<f32x4*>(static_cast<float*>(o) + off) = v;
  }
}

template <int K>
struct alignas(16) P16mem {
  union {
    f16 k[C][K + HP];  // until K K^T is formed
    float t[C][C + PAD];
  };
  float a[C][C + PAD];    // K K^T (upper tiles), then A^T
  float x[32][32 + PAD];  // A21 T11
  float gl[C], bt[C], b[C], gam[C], D[C];
  float gC;
};

// 16-bit inputs: record T diag(beta), P and the gates.  41 KB of LDS at
// K = 128 (k and T share their rows), so four workgroups share a CU.
template <typename TIn, int K>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(K == 64 ? 6 : 8))) void prep16_kernel(const FArgs p) {
  __shared__ P16mem<K> s;
  const int tid = threadIdx.x;
  RowSpan rs;
  int c;
  int64_t ri;
  if (!seg_chunk(p, blockIdx.x, rs, c, ri)) return;
  const int t0 = c * C, nval = min(C, rs.T - t0);
  const int hi = blockIdx.x % p.H;
  float* const rec = p.rec + ri * (int64_t)Rec16::SIZE;
  f16* const rh = reinterpret_cast<f16*>(rec);

  {
    InRows<TIn, C, K, NT> lk;
    lk.load(tid, static_cast<const TIn*>(p.k) + head_base(rs, hi, p.sk) + (int64_t)t0 * p.sk[1], p.sk[1], nval);
    float gv = 0.f, bv = 0.f;
    if (tid < nval) {
      gv = load_scalar(p.g, head_base(rs, hi, p.sg) + (int64_t)(t0 + tid) * p.sg[1], p.g_dtype);
      bv = load_scalar(p.beta, head_base(rs, hi, p.sb) + (int64_t)(t0 + tid) * p.sb[1], p.beta_dtype);
    }
    lk.store(tid, s.k);
    if (tid < C) {
      s.gl[tid] = gv;
      s.bt[tid] = bv;
    }
  }
  __syncthreads();
  chunk_gates(tid, s.gl, s.b, s.gam, s.D, s.gC);
  {
    // K K^T on the 10 tiles on or below the diagonal (exact products, fp32
    // accumulation), each stored transposed, i.e. into the tiles on or above
    // it (K K^T is symmetric): a lane's 4 rows become 4 consecutive columns
    const int lane = tid & 63, r = lane & 15, kq = lane >> 4;
    for (int job = tid >> 6; job < 10; job += NT / 64) {
      const int mt = job < 1 ? 0 : job < 3 ? 1 : job < 6 ? 2 : 3;
      const int nt = job - mt * (mt + 1) / 2;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < K; kb += 32)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag8(&s.k[16 * mt + r][kb + 8 * kq]),
                                                     frag8(&s.k[16 * nt + r][kb + 8 * kq]), acc, 0, 0, 0);
      *reinterpret_cast<f32x4*>(&s.a[16 * nt + r][16 * mt + 4 * kq]) = acc;
    }
  }
  __syncthreads();
  // A^T, A = tril_-1(beta_t M K K^T) (consecutive lanes along a row of A^T)
  for (int e = tid; e < C * C; e += NT) {
    const int j = e / C, t = e % C;
    const float mv = expf(j < t ? s.b[t] - s.b[j] : 0.f);
    s.a[j][t] = j < t ? s.bt[t] * mv * s.a[j][t] : 0.f;
  }
  {
    // P = M o (Q K^T) as fp16 pairs, by tiles of P^T = K Q^T (lane: P[16 tt
    // + r][16 jt + 4 kq + i]): the 10 tiles on or below the diagonal and the
    // two zero tiles above it that the scan's 32-wide products read.  The Q
    // fragments come straight from global memory (rows >= nval read row
    // nval - 1 and are zeroed); the mask is 2^{(b_t - b_j) log2 e} on
    // v_exp_f32 (about 1e-6 relative), 2^{-inf} = 0 above the diagonal.
    const int lane = tid & 63, r = lane & 15, kq = lane >> 4;
    const TIn* const qb = static_cast<const TIn*>(p.q) + head_base(rs, hi, p.sq) + (int64_t)t0 * p.sq[1];
    for (int job = tid >> 6; job < 12; job += NT / 64) {
      const int tt = job < 4 ? job >> 1 : 2 + (job - 4) / 4;
      const int jt = job < 4 ? job & 1 : (job - 4) % 4;
      const int t = 16 * tt + r, j = 16 * jt + 4 * kq;
      const TIn* const qr = qb + (int64_t)min(t, nval - 1) * p.sq[1] + 8 * kq;
      uint4 qv[K / 32];
#pragma unroll
      for (int kb = 0; kb < K / 32; ++kb) qv[kb] = *reinterpret_cast<const uint4*>(qr + 32 * kb);
      f32x4 ap = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < K / 32; ++kb) {
        f16 x[8];
        InTraits<TIn>::to_op(qv[kb], x);
        const f16x8 qf = t < nval ? f16x8{x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]} : f16x8{};
        ap = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag8(&s.k[16 * jt + r][32 * kb + 8 * kq]), qf, ap, 0, 0, 0);
      }
      const float bt = s.b[t];
      f16 h[4], l[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        split_f16(__builtin_amdgcn_exp2f(j + i <= t ? (bt - s.b[j + i]) * 1.44269504f : -__builtin_huge_valf()) *
                      ap[i],
                  h[i], l[i]);
      *reinterpret_cast<f16x4*>(rh + Rec16::PH + t * C + j) = f16x4{h[0], h[1], h[2], h[3]};
      *reinterpret_cast<f16x4*>(rh + Rec16::PL + t * C + j) = f16x4{l[0], l[1], l[2], l[3]};
    }
  }
  if (tid < C) {
    float* const gr = rec + Rec16::GF;
    gr[tid] = s.gam[tid];
    gr[C + tid] = s.D[tid];
    gr[2 * C + tid] = s.b[tid];
    gr[3 * C + tid] = tid == 0 ? s.gC : 0.f;
  }
  __syncthreads();
  solve_t<32 + PAD>(tid, s.a, s.t, s.x);
  // T diag(beta) as fp16 pairs, 8 consecutive entries of a row per lane
  static_assert(C * C == 8 * NT, "one 8-entry piece per lane");
  {
    const int t = tid / 8, j0 = 8 * (tid % 8);
    f16 h[8], l[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) split_f16(s.t[t][j0 + jj] * s.bt[j0 + jj], h[jj], l[jj]);
    *reinterpret_cast<f16x8*>(rh + Rec16::TH + t * C + j0) = f16x8{h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]};
    *reinterpret_cast<f16x8*>(rh + Rec16::TL + t * C + j0) = f16x8{l[0], l[1], l[2], l[3], l[4], l[5], l[6], l[7]};
  }
}

// Row pitches of the scan's LDS arrays (in halves), from LDS bank-conflict
// counters (64 banks of 4 bytes) of each access pattern:
//  * arrays read only as 16-byte operand rows (q, k, T diag(beta), P; k is
//    also read transposed): a pitch of 16 halves past a multiple of 64
//    (8 words past a multiple of 32) gives conflict-free 16-byte row reads;
//  * arrays written in the accumulator layout (8 bytes per lane, lane (r, kq)
//    at row r: S^T, Y^T, u^T, (D u)^T) and read as operand rows: a pitch of
//    4 halves past a multiple of 64 (2 words past a multiple of 32) gives
//    conflict-free 8-byte stores, and the rows are then read by two 8-byte
//    reads (frag8_2; the rows are only 8-byte aligned).  At 8 halves of
//    padding the stores conflicted two ways and the 16-byte reads as well.
template <int K>
constexpr int s16_kq() {
  return (K + 63) / 64 * 64 + 16;
}
template <int K>
struct alignas(16) S16mem {
  static constexpr int KQ = s16_kq<K>(), CQ = C + 16, KS = K + 4, CS = C + 4;
  f16 sh[BV][KS], sl[BV][KS];  // S^T
  f16 q[C][KQ], k[C][KQ];
  f16 th[C][CQ], tl[C][CQ];    // T diag(beta)
  f16 ph[C][CQ], pl[C][CQ];    // P
  f16 vt[BV][CS];              // V^T of the slice
  f16 yh[BV][CS], yl[BV][CS];  // (V - diag(gam) K S)^T
  f16 uh[BV][CS], ul[BV][CS];  // u^T
  f16 dh[BV][CS], dl[BV][CS];  // (diag(D) u)^T
  // gam, D, b, {gam_C, 0 ..}: the record's gate rows, staged by every lane
  // (rows 4 .. 7 repeat them)
  float gv[NT / C][C];
  float ot[4][16][BV + 4];  // o rows of waves 4-7, for vector stores
};

// Next chunk's record and rows, in registers.
template <typename TIn, int K>
struct Next16 {
  HalfRows<C, C, NT> th, tl, ph, pl;
  InRows<TIn, C, K, NT> q, k;
  SlicePairs<TIn, C, BV, NT> v;
  float gate;
  __device__ __forceinline__ void load(const FArgs& p, int tid, int64_t ri, const TIn* qg, const TIn* kg,
                                       const TIn* vg, int t0, int nval) {
    const float* const rec = p.rec + ri * (int64_t)Rec16::SIZE;
    const f16* const rh = reinterpret_cast<const f16*>(rec);
    th.load(tid, rh + Rec16::TH, C);
    tl.load(tid, rh + Rec16::TL, C);
    ph.load(tid, rh + Rec16::PH, C);
    pl.load(tid, rh + Rec16::PL, C);
    q.load(tid, qg + (int64_t)t0 * p.sq[1], p.sq[1], nval);
    k.load(tid, kg + (int64_t)t0 * p.sk[1], p.sk[1], nval);
    v.load(tid, vg + (int64_t)t0 * p.sv[1], p.sv[1], nval);
    gate = rec[Rec16::GF + (tid & (4 * C - 1))];
  }
  __device__ __forceinline__ void store(S16mem<K>& s, int tid, float vsc) const {
    th.store(tid, s.th);
    tl.store(tid, s.tl);
    ph.store(tid, s.ph);
    pl.store(tid, s.pl);
    q.store(tid, s.q);
    k.store(tid, s.k);
    v.store(tid, s.vt, vsc);
    s.gv[tid / C][tid % C] = gate;
  }
};

// Per chunk: (A) K S on waves 0-3 and Q S on waves 4-7 (rows 16 (w & 3) ..),
// then Y = V - diag(gam) K S; (A2) u = T diag(beta) Y on waves 0-3; (B) the
// state update on waves 0-3 while waves 4-7 write o; then the next chunk's
// record and rows are staged.  The fp32 state S lives in the
// accumulators of waves 0-3 (rows 16 (w + 4 j) of K); its hi / lo copies
// in LDS feed K S and Q S.
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
  // this segment's chunks [c0, c0 + nloc) and their records
  const int nloc = max(0, min(p.L, (rs.T + C - 1) / C - p.c0));
  if (nloc == 0 && !p.first) return;  // state unchanged
  const int64_t rb = ((int64_t)bi * p.H + hi) * p.L;
  const TIn* const qg = static_cast<const TIn*>(p.q) + head_base(rs, hi, p.sq);
  const TIn* const kg = static_cast<const TIn*>(p.k) + head_base(rs, hi, p.sk);
  const TIn* const vg = static_cast<const TIn*>(p.v) + head_base(rs, hi, p.sv) + v0;
  const int64_t ob = head_base(rs, hi, p.so) + v0;
  // the state entering the segment: h0 (or zero), or the previous segment's
  const float* const s_in = p.first ? (p.h0 ? p.h0 + bi * p.sh0[0] + hi * p.sh0[1] + v0 * p.sh0[3] : nullptr)
                                    : p.fs + bi * p.sfs[0] + hi * p.sfs[1] + v0 * p.sfs[3];
  const int64_t sik = p.first ? p.sh0[2] : p.sfs[2], siv = p.first ? p.sh0[3] : p.sfs[3];
  // bf16: this segment's rows of the v slice and its entering state scaled
  // into fp16's range, o and the state leaving it scaled back (identity for
  // fp16)
  const int r0 = min(rs.T, p.c0 * C);
  const RangeScale rsc = slice_range_scale<TIn>(
      reinterpret_cast<const char*>(vg + (int64_t)r0 * p.sv[1]), p.sv[1] * (int64_t)sizeof(TIn),
      min(rs.T - r0, nloc * C), BV, s_in, sik, siv, K, p.scale);
  const float scale = rsc.o;

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
        const float x[4] = {st[j][0], st[j][1], st[j][2], st[j][3]};
        store_pair4(&s.sh[r][m0 + 4 * kq], &s.sl[r][m0 + 4 * kq], x);
      }
    }
  };
  if (upper) {
#pragma unroll
    for (int j = 0; j < NST; ++j) {
      const int m0 = 16 * (wave + 4 * j);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st[j][i] = (s_in && m0 < K) ? s_in[(m0 + 4 * kq + i) * sik + r * siv] * rsc.v : 0.f;
    }
    put_state();
  }
  Next16<TIn, K> nx;
  if (nloc > 0) {
    nx.load(p, tid, rb, qg, kg, vg, r0, min(C, rs.T - r0));
    nx.store(s, tid, rsc.v);
  }
  __syncthreads();
  for (int j = 0; j < nloc; ++j) {
    const int t0 = (p.c0 + j) * C, nval = min(C, rs.T - t0);
    // the next chunk's record and rows (the last chunk's again at the end:
    // every load is then consumed by the staging below, on every path)
    const int jn = min(j + 1, nloc - 1), tn = (p.c0 + jn) * C;
    nx.load(p, tid, rb + jn, qg, kg, vg, tn, min(C, rs.T - tn));
    // K S (waves 0-3) or Q S (waves 4-7) for rows um0 ..
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    {
      const f16(*const a)[S16mem<K>::KQ] = upper ? s.k : s.q;
#pragma unroll
      for (int kb = 0; kb < K; kb += 32) {
        const f16x8 af = frag8(&a[um0 + r][kb + 8 * kq]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, frag8_2(&s.sh[r][kb + 8 * kq]), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, frag8_2(&s.sl[r][kb + 8 * kq]), acc, 0, 0, 0);
      }
    }
    if (upper) {
      // Y = V - diag(gam) K S, rows um0 + 4 kq + i, column r, as Y^T pairs
      const int t = um0 + 4 * kq;
      const f16x4 vv = *reinterpret_cast<const f16x4*>(&s.vt[r][t]);
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = (float)vv[i] - s.gv[0][t + i] * acc[i];
      store_pair4(&s.yh[r][t], &s.yl[r][t], y);
    }
    __syncthreads();
    if (upper) {
      // u = T diag(beta) Y for rows um0 .. (T lower triangular: the 32-blocks
      // of columns below um0 + 16)
      f32x4 au = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jb = 0; jb < C; jb += 32)
        if (jb < um0 + 16) {
          const f16x8 th = frag8(&s.th[um0 + r][jb + 8 * kq]), yh = frag8_2(&s.yh[r][jb + 8 * kq]);
          au = __builtin_amdgcn_mfma_f32_16x16x32_f16(th, yh, au, 0, 0, 0);
          au = __builtin_amdgcn_mfma_f32_16x16x32_f16(th, frag8_2(&s.yl[r][jb + 8 * kq]), au, 0, 0, 0);
          au = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag8(&s.tl[um0 + r][jb + 8 * kq]), yh, au, 0, 0, 0);
        }
      // u^T and (diag(D) u)^T as fp16 pairs: lane holds u rows um0 + 4 kq + i, column r
      const int t = um0 + 4 * kq;
      const float u[4] = {au[0], au[1], au[2], au[3]};
      const float du[4] = {s.gv[1][t] * au[0], s.gv[1][t + 1] * au[1], s.gv[1][t + 2] * au[2], s.gv[1][t + 3] * au[3]};
      store_pair4(&s.uh[r][t], &s.ul[r][t], u);
      store_pair4(&s.dh[r][t], &s.dl[r][t], du);
    }
    __syncthreads();
    if (upper) {
      // S <- gam_C S + K^T diag(D) u (K^T read transposed from k)
#pragma unroll
      for (int j = 0; j < NST; ++j) {
        const int m0 = 16 * (wave + 4 * j);
        if (m0 < K) {
          f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int tb = 0; tb < C; tb += 32) {
            const f16x8 kt = frag8_t(s.k, tb, m0, r, kq);
            a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kt, frag8_2(&s.dh[r][tb + 8 * kq]), a, 0, 0, 0);
            a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kt, frag8_2(&s.dl[r][tb + 8 * kq]), a, 0, 0, 0);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) st[j][i] = s.gv[3][0] * st[j][i] + a[i];
        }
      }
      put_state();
    } else {
      // o = scale (P u + diag(gam) Q S)
      f32x4 ao = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jb = 0; jb < C; jb += 32)
        if (jb < um0 + 16) {
          const f16x8 ph = frag8(&s.ph[um0 + r][jb + 8 * kq]), uh = frag8_2(&s.uh[r][jb + 8 * kq]);
          ao = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, uh, ao, 0, 0, 0);
          ao = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph, frag8_2(&s.ul[r][jb + 8 * kq]), ao, 0, 0, 0);
          ao = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag8(&s.pl[um0 + r][jb + 8 * kq]), uh, ao, 0, 0, 0);
        }
      const int row0 = um0 + 4 * kq;
      const f32x4 gm = *reinterpret_cast<const f32x4*>(&s.gv[0][row0]);
      const float ov[4] = {scale * (ao[0] + gm[0] * acc[0]), scale * (ao[1] + gm[1] * acc[1]),
                           scale * (ao[2] + gm[2] * acc[2]), scale * (ao[3] + gm[3] * acc[3])};
      if (p.o_vec) {
        // through this wave's LDS tile: lane -> row lane / 4, columns 4 (lane % 4) ..
        float(*const ot)[BV + 4] = s.ot[wave - 4];
#pragma unroll
        for (int i = 0; i < 4; ++i) ot[4 * kq + i][r] = ov[i];
        const int rr = lane >> 2, c4 = 4 * (lane & 3);
        const f32x4 w = *reinterpret_cast<const f32x4*>(&ot[rr][c4]);
        if (um0 + rr < nval) {
          const int64_t off = ob + (int64_t)(t0 + um0 + rr) * p.so[1] + c4;
          if (p.o_dtype == GDN_DTYPE_F16) store_o_vec4<f16>(p.o, off, w);
          else if (p.o_dtype == GDN_DTYPE_BF16) store_o_vec4<bf16_t>(p.o, off, w);
          else store_o_vec4<float>(p.o, off, w);
        }
      } else {
        const int64_t base = ob + (int64_t)(t0 + row0) * p.so[1] + r;
        if (p.o_dtype == GDN_DTYPE_F16) store_o4<f16>(p.o, base, p.so[1], nval - row0, ov);
        else if (p.o_dtype == GDN_DTYPE_BF16) store_o4<bf16_t>(p.o, base, p.so[1], nval - row0, ov);
        else store_o4<float>(p.o, base, p.so[1], nval - row0, ov);
      }
    }
    __syncthreads();
    nx.store(s, tid, rsc.v);
    __syncthreads();
  }
  if (upper) {
#pragma unroll
    for (int j = 0; j < NST; ++j) {
      const int m0 = 16 * (wave + 4 * j);
      if (m0 < K) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          p.fs[bi * p.sfs[0] + hi * p.sfs[1] + (m0 + 4 * kq + i) * p.sfs[2] + (v0 + r) * p.sfs[3]] = st[j][i] * rsc.fs;
      }
    }
  }
}

template <typename TIn, int K>
int launch_k(const FArgs& a, int64_t nrec, hipStream_t s) {
  if constexpr (std::is_same<TIn, float>::value) {
    if (nrec > 0) hipLaunchKernelGGL((prep_kernel<K>), dim3((unsigned)nrec), dim3(NT), 0, s, a);
    hipLaunchKernelGGL((scan_kernel<TIn, K>), dim3(a.units), dim3(NT), 0, s, a);
  } else {
    if (nrec > 0) hipLaunchKernelGGL((prep16_kernel<TIn, K>), dim3((unsigned)nrec), dim3(NT), 0, s, a);
    hipLaunchKernelGGL((scan16_kernel<TIn, K>), dim3(a.units), dim3(NT), 0, s, a);
  }
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

// Bytes of one record (chunk, head) for this input dtype.
int64_t c64_record_bytes(int K, int qkv_dtype) { return c64::rec_floats(K, qkv_dtype != GDN_DTYPE_F32) * 4; }

// Records of min(ceil(T / C), kSegC64) chunks per (sequence, head), in bytes:
// longer sequences run in segments of that many chunks.
int64_t c64_workspace_size(int B, int T, int H, int K, int n_seq, int qkv_dtype) {
  const int64_t nch = (T + c64::C - 1) / c64::C;
  const int64_t L = nch < kSegC64 ? nch : kSegC64;
  const int64_t nseq = n_seq > 0 ? n_seq : B;
  return c64::align256(nseq * H * L * c64_record_bytes(K, qkv_dtype));
}

bool c64_supported(int K, int C, int V) { return C == c64::C && (K == 32 || K == 64 || K == 128) && V % 16 == 0; }

// Enqueue the (prep, scan) launches of every segment of seg_chunks chunks
// (arguments, and a workspace of B * H * seg_chunks records, checked by the
// caller).
int c64_launch(const GdnFwdParams& P, int seg_chunks, hipStream_t stream) {
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
  {
    const int64_t vb = 4 * (P.o_dtype == GDN_DTYPE_F32 ? 4 : 2);  // bytes of a 4-element store
    const int64_t eb = vb / 4;
    a.o_vec = reinterpret_cast<uintptr_t>(P.o) % vb == 0 && (P.o_stride[0] * eb) % vb == 0 &&
              (P.o_stride[1] * eb) % vb == 0 && (P.o_stride[2] * eb) % vb == 0;
  }
  // every sequence has at most ceil(T / C) chunks (the offsets are not read here)
  const int L = a.nchmax > 0 ? (seg_chunks < a.nchmax ? seg_chunks : a.nchmax) : 1;
  const int nseg = a.nchmax > 0 ? (a.nchmax + L - 1) / L : 1;
  const int64_t nrec = a.nchmax > 0 ? (int64_t)P.B * P.H * L : 0;
  if (nrec > 0x7fffffffLL) return GDN_ERR_BAD_SHAPE;
  a.L = L;
  for (int sg = 0; sg < nseg; ++sg) {
    a.c0 = sg * L;
    a.first = sg == 0;
    int st;
    switch (P.qkv_dtype) {
      case GDN_DTYPE_F16: st = c64::launch_t<f16>(a, P.K, nrec, stream); break;
      case GDN_DTYPE_BF16: st = c64::launch_t<bf16_t>(a, P.K, nrec, stream); break;
      default: st = c64::launch_t<float>(a, P.K, nrec, stream); break;
    }
    if (st != 0) return st;
  }
  return GDN_OK;
}

}  // namespace gdn
