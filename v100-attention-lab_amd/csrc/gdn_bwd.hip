// Backward of the chunked GDN forward: gradients of q, k, v, g, beta, h0.
//
// Per chunk (C = 32 rows, within-chunk gate cumsum b, gam = e^b, D_j =
// e^{bC - b_j}, M[t][j] = e^{b_t - b_j} for j <= t) the forward is
//   A = tril_-1(beta_t M KK^T), T = (I + A)^-1,
//   W = T diag(beta gam) K,  U = T diag(beta) V,  u = U - W S,
//   o = scale (M o (Q K^T)) u + scale diag(gam) Q S,
//   S' = gam_C S + K^T diag(D) u,
// and its reverse-mode derivative, given dO and dS' (the gradient of S'), is
//   du  = scale P^T dO + diag(D) K dS'            (P = M o Q K^T)
//   dQK = M o (scale dO u^T)
//   dW  = -du S^T,  dT = du (diag(beta) V)^T + dW (diag(beta gam) K)^T
//   dW~ = T^T dW,   dU~ = T^T du,   dA = -tril_-1(T^T dT T^T)
//   dq  = dQK K + scale diag(gam) dO S^T
//   dk  = dQK^T Q + diag(D) u dS'^T + diag(beta gam) dW~ + (dKK + dKK^T) K,
//         dKK = dA o beta_t M
//   dv  = diag(beta) dU~
//   dbeta_t = v_t.dU~_t + gam_t k_t.dW~_t + sum_j dA M KK
//   db: through gam, gam_C, D, M and A; dg = reverse cumsum of db
//   dS  = scale Q^T diag(gam) dO + gam_C dS' - W^T du   (dS' of the chunk before)
// (checked against reverse-mode differentiation of the step recurrence
// gdn_ref.py:3-9).  Two row sums are taken from C x K products instead of
// C x V ones: u_t.(K dS')_t = k_t.(u dS'^T)_t and dO_t.(Q S)_t =
// q_t.(dO S^T)_t.
//
// Only S (forward) and dS (backward) carry from chunk to chunk, and each
// needs a few products per chunk; everything else is independent per chunk.
// So the backward is three launches, on the fp32 matrix cores
// (v_mfma_f32_16x16x4_f32) except the 16-bit recurrences:
//   1. prep_kernel, one workgroup per (chunk, head): gates, K K^T, P, T and
//      (fp32 only) W, written once to a per-chunk record (the
//      state-independent half of the chunk's forward, shared by every
//      V-slice below), and for 16-bit inputs T diag(beta) and P as fp16
//      pairs as well;
//   2. recur_kernel (fp32) or recur16_kernel (16-bit q, k, v, dO: fp16 MFMA
//      on hi + lo pairs), one workgroup per (sequence, head, 16-column V
//      slice) and direction, both directions in one launch: the forward
//      walk stores each chunk's start state S and u; the backward walk
//      stores each chunk's dS' and du and finally dh0.  The 16-bit walks
//      store S and dS' in fp16 (half the bytes of the largest arrays of
//      the backward), in their range-shifted units with one scale per
//      walk;
//   3. grad_kernel, one workgroup per (chunk, head) over all of V: every
//      gradient of the chunk from the stored S, dS', u, du and the record,
//      written directly in the output dtypes (V is walked in 32-column steps,
//      16 when V is an odd multiple of 16, with the C x K products held in
//      MFMA accumulators).
// Packed sequences (cu_seqlens): sequence i owns chunk slots floor(t0 / C) +
// i onwards, one per chunk; the ranges are disjoint, so every launch handles
// packed sequences like a batch.

#include "gdn_fwd_pipe.h"
#include "gdn_tiles_f16.h"

namespace gdn {
namespace bwd {

using namespace tiles;

constexpr int C = 32;
constexpr int BV = 16;    // state columns per workgroup of the recurrences
constexpr int NTP = 256;  // threads: prep_kernel and recur_kernel (4 waves)
constexpr int NTG = 512;  // threads: grad_kernel (8 waves)

struct BArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  const float* h0;
  const void* d_o;
  const float* dfs;
  void* dq;
  void* dk;
  void* dv;
  void* dg;
  void* dbeta;
  float* dh0;
  float* rec;  // per (slot, head): the prep kernel's record
  // per (slot, head): S at the chunk start and dS', the gradient of the
  // state after the chunk: fp32 [K][V], or from the 16-bit walks fp16 [V][K]
  // (rows = state columns, in each walk's range-shifted units: scl below
  // scales them back)
  float* ckS;
  float* ckD;
  float* uu;   // per (slot, head): u, [C][V]
  float* du;   // per (slot, head): du, [C][V]
  f16* r16;    // per (slot, head): T diag(beta) and P as fp16 pairs (16-bit walks)
  float* scl;  // per walk unit (sequence, head, V-slice): the power of two that
               // takes the fp16 ckS (units first) and ckD (then) back to true units
  int w16;     // the recurrences run on fp16 pairs (16-bit q, k, v and dO)
  int64_t sq[3], sk[3], sv[3], sg[3], sb[3], sdo[3], sdq[3], sdk[3], sdv[3], sdg[3], sdb[3];
  int64_t sh0[4], sdfs[4], sdh0[4];
  int B, T, H, V, nv, nchmax, units;
  float scale;
  int g_dtype, beta_dtype, do_dtype;
  const int64_t* cu;
  int xcd_remap;
};

// Per-(slot, head) record, in floats: T, P = M o Q K^T and K K^T as [C][C],
// W as [C][K], then b, gam, D as [C] each and gam_C (first of a [C] row).
template <int K>
struct Rec {
  static constexpr int T = 0, PM = C * C, KK = 2 * C * C, W = 3 * C * C;
  static constexpr int G = W + C * K;
  static constexpr int SIZE = G + 4 * C;
};
inline int64_t rec_size(int K) { return 3 * C * C + (int64_t)C * K + 4 * C; }
// The 16-bit walks' per-(slot, head) record, in floats: T as [C][C], then
// the gates as in Rec (their products take P, K K^T and W from elsewhere).
struct RecT {
  static constexpr int T = 0, G = C * C;
  static constexpr int SIZE = G + 4 * C;
};
// The same chunk's operands of the 16-bit recurrences, in halves: T diag(beta)
// and P as [C][C], each an fp16 pair hi + lo.
struct Rec16 {
  static constexpr int TBH = 0, TBL = C * C, PH = 2 * C * C, PL = 3 * C * C;
  static constexpr int SIZE = 4 * C * C;
};
inline int64_t rec16_size(int) { return 4 * C * C; }

// ---------------------------------------------------------------------------
// 1. prep: the state-independent half of a chunk's forward
// ---------------------------------------------------------------------------

template <int K>
struct alignas(16) PSmem {
  float q[C][K + 1], k[C][K + 1];
  float kk[C][C + 1], qk[C][C + 1], a[C][C + 1], t[C][C + 1];
  float gl[C], bt[C], b[C], gam[C], D[C];
  float gC;
};

template <typename TIn, int K>
__global__ __launch_bounds__(NTP) void prep_kernel(const BArgs p) {
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
  f16* const rh = p.r16 + (slot * p.H + hi) * (int64_t)Rec16::SIZE;

  {
    RowLoad<TIn, C, K, NTP> lq, lk;
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
    mmx<NTP, C, C>(tid, [&](int m, int n, float x) { s.kk[m][n] = x; },
                   seg<K>([&](int m, int kk) { return s.k[m][kk]; }, [&](int kk, int n) { return s.k[n][kk]; }));
    mmx<NTP, C, C>(tid, [&](int m, int n, float x) { s.qk[m][n] = x; },
                   seg<K>([&](int m, int kk) { return s.q[m][kk]; }, [&](int kk, int n) { return s.k[n][kk]; }));
  } else {
    // 16-bit q and k are exact in fp16: K K^T and Q K^T on
    // v_mfma_f32_16x16x32_f16 (exact products, fp32 accumulation), the 8
    // tiles over the 4 waves
    const int lane = tid & 63, r = lane & 15, kq = lane >> 4;
    auto frag = [](const float* row) __attribute__((always_inline)) {
      f16x8 f;
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (f16)row[e];
      return f;
    };
    for (int job = tid >> 6; job < 8; job += NTP / 64) {
      const int mat = job >> 2, mt = (job >> 1) & 1, nt = job & 1;
      const float* const arow = (mat ? &s.q[0][0] : &s.k[0][0]) + (16 * mt + r) * (K + 1) + 8 * kq;
      const float* const brow = &s.k[0][0] + (16 * nt + r) * (K + 1) + 8 * kq;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < K; kb += 32)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag(arow + kb), frag(brow + kb), acc, 0, 0, 0);
      float(*const dst)[C + 1] = mat ? s.qk : s.kk;
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[16 * mt + 4 * kq + i][16 * nt + r] = acc[i];
    }
  }
  __syncthreads();
  for (int e = tid; e < C * C; e += NTP) {
    const int t = e / C, j = e % C;
    const float mv = j <= t ? expf(s.b[t] - s.b[j]) : 0.f;
    s.a[t][j] = j < t ? s.bt[t] * mv * s.kk[t][j] : 0.f;
    rec[R::PM + e] = mv * s.qk[t][j];
    rec[R::KK + e] = s.kk[t][j];
    if (p.w16) tiles16::split_f16(mv * s.qk[t][j], rh[Rec16::PH + e], rh[Rec16::PL + e]);
  }
  if (tid < C) {
    rec[R::G + tid] = s.b[tid];
    rec[R::G + C + tid] = s.gam[tid];
    rec[R::G + 2 * C + tid] = s.D[tid];
    rec[R::G + 3 * C + tid] = tid == 0 ? s.gC : 0.f;
  }
  __syncthreads();
  if (tid < C) {
    // column tid of T = (I + A)^-1 by forward substitution, in registers
    const int cc = tid;
    float col[C];
#pragma unroll
    for (int i = 0; i < C; ++i) {
      float x = (i == cc) ? 1.f : 0.f;
#pragma unroll
      for (int j = 0; j < i; ++j) x = __builtin_fmaf(-s.a[i][j], col[j], x);
      col[i] = x;
    }
#pragma unroll
    for (int i = 0; i < C; ++i) {
      s.t[i][cc] = col[i];
      rec[R::T + i * C + cc] = col[i];
    }
  }
  __syncthreads();
  // the 16-bit recurrences' operand T diag(beta) as fp16 pairs, 4 entries
  // per lane
  if (p.w16) {
    static_assert(C * C == 4 * NTP, "4 entries of T per lane");
    const int t = tid / (C / 4), j0 = 4 * (tid % (C / 4));
    f16 h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) tiles16::split_f16(s.t[t][j0 + i] * s.bt[j0 + i], h[i], l[i]);
    *reinterpret_cast<f16x4*>(rh + Rec16::TBH + t * C + j0) = f16x4{h[0], h[1], h[2], h[3]};
    *reinterpret_cast<f16x4*>(rh + Rec16::TBL + t * C + j0) = f16x4{l[0], l[1], l[2], l[3]};
  }
  // W = T diag(beta gam) K, read by the fp32 recurrences only
  if (!p.w16)
    mmx<NTP, C, K>(tid, [&](int m, int n, float x) { rec[R::W + m * K + n] = x; },
                   seg<C>([&](int m, int kk) { return s.t[m][kk]; },
                          [&](int kk, int n) { return s.bt[kk] * s.gam[kk] * s.k[kk][n]; }));
}

// 16-bit q or k rows as MFMA operands: 8 elements (16 bytes) per lane, in
// their own type (exact), on v_mfma_f32_16x16x32_f16 or _bf16.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
template <typename TIn>
__device__ __forceinline__ f32x4 mma16(const u32x4& a, const u32x4& b, const f32x4& acc) {
  if constexpr (std::is_same<TIn, f16>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), acc, 0,
                                                  0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc,
                                                   0, 0, 0);
}
// 8 consecutive fp32 values that hold 16-bit inputs, back in their own type
// (exact).
template <typename TIn>
__device__ __forceinline__ u32x4 pack16(const float* x) {
  u32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (std::is_same<TIn, f16>::value) {
      const f16 lo = (f16)x[2 * e], hi = (f16)x[2 * e + 1];
      r[e] = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    } else {
      r[e] = (__float_as_uint(x[2 * e]) >> 16) | (__float_as_uint(x[2 * e + 1]) & 0xffff0000u);
    }
  }
  return r;
}

// The prep of the 16-bit recurrences: one wave per two (chunk, head)
// records, with no workgroup barrier.  Per record: the gates (a prefix sum
// across lanes), K K^T and Q K^T on the 16-bit matrix cores (exact
// products, fp32 sums), A = beta_t e^{b_t - b_j} K K^T (t > j) staged as
// A^T in the wave's LDS, then T = (I + A)^-1 by substitution with one lane
// per row of T (lanes 0-31: record 0, lanes 32-63: record 1).  It writes T
// and the gates to the fp32 record, and T diag(beta) and P = M o Q K^T as
// fp16 pairs; the gradient kernel forms P and K K^T in fp32 itself (from
// the q and k rows it loads anyway), so they are not written here.  Rows
// past a chunk's end read the last row again: their beta and gate are
// zero, which zeroes their rows of A and T (and their rows of P are
// zeroed), so the record equals that of zero rows.
constexpr int NRW = 2;  // records per wave

template <typename TIn, int K>
__global__ __launch_bounds__(256) void prep16_kernel(const BArgs p, int64_t nrec) {
  using R = RecT;
  constexpr int KB = K / 32;
  __shared__ __attribute__((aligned(16))) float s_at[4][NRW][C * C];  // A^T row-major
  __shared__ __attribute__((aligned(16))) float s_beta[4][NRW][C];
  __shared__ __attribute__((aligned(16))) float s_b[4][NRW][C];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, gq = lane >> 4;
  const int half = lane >> 5, c = lane & 31;

  // the records of this wave (wave-uniform)
  int nval[NRW];
  const TIn* qh[NRW];
  const TIn* kh[NRW];
  int64_t gb[NRW], bb[NRW], ri[NRW];
#pragma unroll
  for (int e = 0; e < NRW; ++e) {
    const int64_t rid = ((int64_t)blockIdx.x * 4 + wave) * NRW + e;
    nval[e] = 0;
    qh[e] = kh[e] = nullptr;
    gb[e] = bb[e] = ri[e] = 0;
    RowSpan rs;
    int cc;
    if (rid < nrec && slot_chunk<C>(p, rid / p.H, rs, cc)) {
      const int hi = (int)(rid % p.H), t0 = cc * C;
      nval[e] = min(C, rs.T - t0);
      qh[e] = static_cast<const TIn*>(p.q) + head_base(rs, hi, p.sq) + (int64_t)t0 * p.sq[1];
      kh[e] = static_cast<const TIn*>(p.k) + head_base(rs, hi, p.sk) + (int64_t)t0 * p.sk[1];
      gb[e] = head_base(rs, hi, p.sg) + (int64_t)t0 * p.sg[1];
      bb[e] = head_base(rs, hi, p.sb) + (int64_t)t0 * p.sb[1];
      ri[e] = rid;
    }
  }
  // q and k rows as operand fragments: lane (n, gq) holds row 16 mt + n,
  // columns 32 kb + 8 gq .. + 7
  u32x4 qr[NRW][2][KB], kr[NRW][2][KB];
#pragma unroll
  for (int e = 0; e < NRW; ++e) {
    if (nval[e] > 0) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int64_t row = min(16 * mt + n, nval[e] - 1);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          kr[e][mt][kb] = *reinterpret_cast<const u32x4*>(kh[e] + row * p.sk[1] + 32 * kb + 8 * gq);
          qr[e][mt][kb] = *reinterpret_cast<const u32x4*>(qh[e] + row * p.sq[1] + 32 * kb + 8 * gq);
        }
      }
    }
  }
  // gates of row c of record `half`
  float gv = 0.f, bv = 0.f;
  {
    const int nv = half ? nval[1] : nval[0];
    if (c < nv) {
      gv = load_scalar(p.g, (half ? gb[1] : gb[0]) + (int64_t)c * p.sg[1], p.g_dtype);
      bv = load_scalar(p.beta, (half ? bb[1] : bb[0]) + (int64_t)c * p.sb[1], p.beta_dtype);
    }
  }
  const float b = pipe::scan32(gv);
  const float bC0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(b), 31));
  const float bC1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(b), 63));
  const float bC = half ? bC1 : bC0;
  s_beta[wave][half][c] = bv;
  s_b[wave][half][c] = b;
  float* const rec_h = p.rec + (half ? ri[1] : ri[0]) * (int64_t)R::SIZE;
  if ((half ? nval[1] : nval[0]) > 0) {
    rec_h[R::G + c] = b;
    rec_h[R::G + C + c] = expf(b);
    rec_h[R::G + 2 * C + c] = expf(bC - b);
    rec_h[R::G + 3 * C + c] = c == 0 ? expf(bC) : 0.f;
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

#pragma unroll
  for (int e = 0; e < NRW; ++e) {
    if (nval[e] > 0) {
      const float* const sb = s_b[wave][e];
      // A^T from the lower tiles of K K^T (the upper one is never read)
      float* const sa = s_at[wave][e];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt <= mt; ++nt) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) acc = mma16<TIn>(kr[e][mt][kb], kr[e][nt][kb], acc);
          // acc[i] = (K K^T)[t = 16 mt + 4 gq + i][j = 16 nt + n]
          const int jj = 16 * nt + n;
          const float bj = sb[jj];
          const f32x4 bt4 = *reinterpret_cast<const f32x4*>(&sb[16 * mt + 4 * gq]);
          const f32x4 be4 = *reinterpret_cast<const f32x4*>(&s_beta[wave][e][16 * mt + 4 * gq]);
          f32x4 av;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int t = 16 * mt + 4 * gq + i;
            av[i] = t > jj ? be4[i] * expf(bt4[i] - bj) * acc[i] : 0.f;
          }
          *reinterpret_cast<f32x4*>(sa + jj * C + 16 * mt + 4 * gq) = av;
        }
      // P = M o Q K^T as fp16 pairs, row-major: the product K Q^T puts 4
      // consecutive columns of one row of P in each lane
      f16* const rh = p.r16 + ri[e] * (int64_t)Rec16::SIZE;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int t = 16 * mt + n;
        const float btv = sb[t];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          f16 h[4] = {(f16)0.f, (f16)0.f, (f16)0.f, (f16)0.f}, l[4] = {h[0], h[1], h[2], h[3]};
          if (nt <= mt) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) acc = mma16<TIn>(kr[e][nt][kb], qr[e][mt][kb], acc);
            const f32x4 bj4 = *reinterpret_cast<const f32x4*>(&sb[16 * nt + 4 * gq]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int j = 16 * nt + 4 * gq + i;
              const float x = (j <= t && t < nval[e]) ? expf(btv - bj4[i]) * acc[i] : 0.f;
              tiles16::split_f16(x, h[i], l[i]);
            }
          }
          const int off = t * C + 16 * nt + 4 * gq;
          *reinterpret_cast<f16x4*>(rh + Rec16::PH + off) = f16x4{h[0], h[1], h[2], h[3]};
          *reinterpret_cast<f16x4*>(rh + Rec16::PL + off) = f16x4{l[0], l[1], l[2], l[3]};
        }
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

  // row c of T of record `half`: xc[i] = T[c][i]
  float xc[C];
#pragma unroll
  for (int i = 0; i < C; ++i) xc[i] = 0.f;
  const float* const at = s_at[wave][half];
  pipe::solve_rows<19, 32>(at, c, xc);
  pipe::solve_rows<13, 19>(at, c, xc);
  pipe::solve_rows<9, 13>(at, c, xc);
  pipe::solve_rows1<6, 9>(at, c, xc);
  pipe::solve_rows1<3, 6>(at, c, xc);
  pipe::solve_rows1<0, 3>(at, c, xc);
  if ((half ? nval[1] : nval[0]) > 0) {
    float* const tr = rec_h + R::T + c * C;
#pragma unroll
    for (int i = 0; i < C; i += 4) *reinterpret_cast<f32x4*>(tr + i) = f32x4{xc[i], xc[i + 1], xc[i + 2], xc[i + 3]};
    // row c of T diag(beta) as fp16 pairs
    f16* const rh = p.r16 + (half ? ri[1] : ri[0]) * (int64_t)Rec16::SIZE + c * C;
    const float* const be = s_beta[wave][half];
#pragma unroll
    for (int j = 0; j < C; j += 8) {
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(be + j), b1 = *reinterpret_cast<const f32x4*>(be + j + 4);
      f16x8 h, l;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f16 hh, ll;
        tiles16::split_f16(xc[j + i] * b0[i], hh, ll);
        h[i] = hh;
        l[i] = ll;
        tiles16::split_f16(xc[j + 4 + i] * b1[i], hh, ll);
        h[4 + i] = hh;
        l[4 + i] = ll;
      }
      *reinterpret_cast<f16x8*>(rh + Rec16::TBH + j) = h;
      *reinterpret_cast<f16x8*>(rh + Rec16::TBL + j) = l;
    }
  }
}

// ---------------------------------------------------------------------------
// 2. the two recurrences (one launch: blocks [0, units) walk forward, the
//    rest backward)
//
// Per chunk each walk needs one product through the carried state and one
// that updates it.  The first (u or du: two 16 x 16 tiles, contraction
// C + K) is split over the four waves by contraction range and the partial
// tiles summed once, so that every wave works in both products.  The chunk's record and input rows for the next
// chunk are loaded into registers while the current chunk computes.
// ---------------------------------------------------------------------------

constexpr int NWP = NTP / 64;  // waves of a recurrence workgroup

template <int K>
struct alignas(16) FSmem {
  float S[K][BV + 1];
  float t[C][C + 1];
  float w[C][K + 1], k[C][K + 1];
  float v[C][BV + 1], u[C][BV + 1];
  float part[NWP][C][BV + 1];  // partial u tiles, one per wave
  float bt[C], D[C];
  float gC;
};

template <int K>
struct alignas(16) RSmem {
  float dS[K][BV + 1];
  float pm[C][C + 1];
  float q[C][K + 1], k[C][K + 1], w[C][K + 1];
  float dO[C][BV + 1], du[C][BV + 1];
  float part[NWP][C][BV + 1];  // partial du tiles, one per wave
  float gam[C], D[C];
  float gC;
};

template <int K>
union FRSmem {
  FSmem<K> f;
  RSmem<K> r;
};

// acc[g] += sum over kc in [kc0, kc0 + LEN) of a(m, kc) b(kc, n) for the two
// C x 16 tiles (rows 0-15, 16-31), where kc < C1 takes (a1, b1) at kc and
// kc >= C1 takes (a2, b2) at kc - C1.  kc0 is wave-uniform, so the two
// loops have uniform bounds and no per-lane branches.
template <int LEN, int C1, typename FA1, typename FB1, typename FA2, typename FB2>
__device__ __forceinline__ void split_tiles(f32x4 (&acc)[2], int kc0, int r, int kq, FA1&& a1, FB1&& b1,
                                            FA2&& a2, FB2&& b2) {
  static_assert(LEN % 4 == 0 && C1 % 4 == 0, "contraction steps");
  const int e1 = min(kc0 + LEN, C1);
  for (int k0 = kc0; k0 < e1; k0 += 4) {
    const float b0 = b1(k0 + kq, r);
    acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1(r, k0 + kq), b0, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1(16 + r, k0 + kq), b0, acc[1], 0, 0, 0);
  }
  for (int k0 = max(kc0, C1) - C1; k0 < kc0 + LEN - C1; k0 += 4) {
    const float b0 = b2(k0 + kq, r);
    acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a2(r, k0 + kq), b0, acc[0], 0, 0, 0);
    acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a2(16 + r, k0 + kq), b0, acc[1], 0, 0, 0);
  }
}

// K x BV state block (LDS) -> rows of a [K][V] fp32 array, 16 bytes per
// store.  A fixed count of stores per thread (no loop over a thread-dependent
// range), so that waits for loads issued before them need not wait for them.
template <int K>
__device__ __forceinline__ void store_state(int tid, const float (*st)[BV + 1], float* dst, int64_t ld) {
  constexpr int NV = K * BV / 4, PER = (NV + NTP - 1) / NTP;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = tid + i * NTP;
    if (NV % NTP == 0 || e < NV) {
      const int kk = e / (BV / 4), c4 = (e % (BV / 4)) * 4;
      *reinterpret_cast<f32x4*>(dst + kk * ld + c4) = f32x4{st[kk][c4], st[kk][c4 + 1], st[kk][c4 + 2], st[kk][c4 + 3]};
    }
  }
}

// Next chunk's state-independent inputs of the forward walk, in registers.
template <typename TIn, int K>
struct FNext {
  RowLoad<float, C, C, NTP> lt;
  RowLoad<float, C, K, NTP> lw;
  RowLoad<TIn, C, K, NTP> lk;
  RowLoad<TIn, C, BV, NTP> lv;
  uint32_t bv;
  float dv, gc;
  __device__ __forceinline__ void load(const BArgs& p, int tid, int64_t ri, const TIn* kg, const TIn* vg,
                                       int64_t bb, int t0, int nval) {
    using R = Rec<K>;
    const float* const rec = p.rec + ri * R::SIZE;
    lt.load(tid, rec + R::T, C, C);
    lw.load(tid, rec + R::W, K, C);
    lk.load(tid, kg + (int64_t)t0 * p.sk[1], p.sk[1], nval);
    lv.load(tid, vg + (int64_t)t0 * p.sv[1], p.sv[1], nval);
    bv = (tid < nval) ? load_bits(p.beta, bb + (int64_t)(t0 + tid) * p.sb[1], p.beta_dtype) : 0u;
    dv = tid < C ? rec[R::G + 2 * C + tid] : 0.f;
    gc = tid == 0 ? rec[R::G + 3 * C] : 0.f;
  }
  __device__ __forceinline__ void store(FSmem<K>& s, int tid, int beta_dtype) const {
    lt.store(tid, s.t);
    lw.store(tid, s.w);
    lk.store(tid, s.k);
    lv.store(tid, s.v);
    if (tid < C) {
      s.bt[tid] = bits_to_float(bv, beta_dtype);
      s.D[tid] = dv;
    }
    if (tid == 0) s.gC = gc;
  }
};

// Forward walk: S at each chunk start -> ckS, u -> uu.
template <typename TIn, int K>
__device__ __forceinline__ void walk_forward(const BArgs& p, FSmem<K>& s, const RowSpan& rs, int bi, int hi,
                                             int v0, int64_t slot0) {
  constexpr int LEN = (C + K) / NWP;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, kq = lane >> 4;
  const int nch = (rs.T + C - 1) / C;
  const TIn* const kg = static_cast<const TIn*>(p.k) + head_base(rs, hi, p.sk);
  const TIn* const vg = static_cast<const TIn*>(p.v) + head_base(rs, hi, p.sv) + v0;
  const int64_t bb = head_base(rs, hi, p.sb);
  for (int e = tid; e < K * BV; e += NTP) {
    const int kk = e / BV, c2 = e % BV;
    s.S[kk][c2] = p.h0 ? p.h0[bi * p.sh0[0] + hi * p.sh0[1] + kk * p.sh0[2] + (v0 + c2) * p.sh0[3]] : 0.f;
  }
  FNext<TIn, K> nx;
  if (nch > 0) {
    nx.load(p, tid, slot0 * p.H + hi, kg, vg, bb, 0, min(C, rs.T));
    nx.store(s, tid, p.beta_dtype);
  }
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    const int64_t ri = (slot0 + c) * p.H + hi;
    if (c + 1 < nch) nx.load(p, tid, ri + p.H, kg, vg, bb, (c + 1) * C, min(C, rs.T - (c + 1) * C));
    float* const cks = p.ckS + ri * (int64_t)K * p.V + v0;
    float* const uo = p.uu + ri * (int64_t)C * p.V + v0;
    store_state<K>(tid, s.S, cks, p.V);
    // partial u = [T, -W] [diag(beta) V; S] over this wave's contraction range
    {
      f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
      split_tiles<LEN, C>(
          acc, wave * LEN, r, kq, [&](int m, int kk) { return s.t[m][kk]; },
          [&](int kk, int n) { return s.bt[kk] * s.v[kk][n]; }, [&](int m, int kk) { return -s.w[m][kk]; },
          [&](int kk, int n) { return s.S[kk][n]; });
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s.part[wave][4 * kq + i][r] = acc[0][i];
        s.part[wave][16 + 4 * kq + i][r] = acc[1][i];
      }
    }
    __syncthreads();
    // u = the sum of the partial tiles, once
#pragma unroll
    for (int i = 0; i < C * BV / NTP; ++i) {
      const int e = tid + i * NTP, m = e / BV, n = e % BV;
      float x = s.part[0][m][n];
#pragma unroll
      for (int w = 1; w < NWP; ++w) x += s.part[w][m][n];
      s.u[m][n] = x;
      uo[(int64_t)m * p.V + n] = x;
    }
    __syncthreads();
    // S <- gam_C S + K^T diag(D) u
    mmx<NTP, K, BV>(tid, [&](int m, int n, float x) { s.S[m][n] = s.gC * s.S[m][n] + x; },
                    seg<C>([&](int m, int kk) { return s.k[kk][m] * s.D[kk]; },
                           [&](int kk, int n) { return s.u[kk][n]; }));
    __syncthreads();
    if (c + 1 < nch) {
      nx.store(s, tid, p.beta_dtype);
      __syncthreads();
    }
  }
}

// Next chunk's state-independent inputs of the backward walk, in registers.
template <typename TIn, int K>
struct RNext {
  static constexpr int NDO = C * BV / NTP;
  static_assert(C * BV % NTP == 0, "dO elements per thread");
  RowLoad<float, C, C, NTP> lp;
  RowLoad<float, C, K, NTP> lw;
  RowLoad<TIn, C, K, NTP> lq, lk;
  uint32_t rdo[NDO];
  float gm, dv, gc;
  __device__ __forceinline__ void load(const BArgs& p, int tid, int64_t ri, const TIn* qg, const TIn* kg,
                                       int64_t dob, int t0, int nval) {
    using R = Rec<K>;
    const float* const rec = p.rec + ri * R::SIZE;
    lp.load(tid, rec + R::PM, C, C);
    lw.load(tid, rec + R::W, K, C);
    lq.load(tid, qg + (int64_t)t0 * p.sq[1], p.sq[1], nval);
    lk.load(tid, kg + (int64_t)t0 * p.sk[1], p.sk[1], nval);
#pragma unroll
    for (int i = 0; i < NDO; ++i) {
      const int e = tid + i * NTP, t = e / BV, c2 = e % BV;
      rdo[i] = t < nval ? load_bits(p.d_o, dob + (int64_t)(t0 + t) * p.sdo[1] + c2, p.do_dtype) : 0u;
    }
    gm = tid < C ? rec[R::G + C + tid] : 0.f;
    dv = tid < C ? rec[R::G + 2 * C + tid] : 0.f;
    gc = tid == 0 ? rec[R::G + 3 * C] : 0.f;
  }
  __device__ __forceinline__ void store(RSmem<K>& s, int tid, int do_dtype) const {
    lp.store(tid, s.pm);
    lw.store(tid, s.w);
    lq.store(tid, s.q);
    lk.store(tid, s.k);
#pragma unroll
    for (int i = 0; i < NDO; ++i) {
      const int e = tid + i * NTP;
      s.dO[e / BV][e % BV] = bits_to_float(rdo[i], do_dtype);
    }
    if (tid < C) {
      s.gam[tid] = gm;
      s.D[tid] = dv;
    }
    if (tid == 0) s.gC = gc;
  }
};

// Backward walk: dS' of each chunk -> ckD, du -> du, at the end dh0.
template <typename TIn, int K>
__device__ __forceinline__ void walk_backward(const BArgs& p, RSmem<K>& s, const RowSpan& rs, int bi, int hi,
                                              int v0, int64_t slot0) {
  constexpr int LEN = (C + K) / NWP;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, kq = lane >> 4;
  const int nch = (rs.T + C - 1) / C;
  const float scale = p.scale;
  const TIn* const qg = static_cast<const TIn*>(p.q) + head_base(rs, hi, p.sq);
  const TIn* const kg = static_cast<const TIn*>(p.k) + head_base(rs, hi, p.sk);
  const int64_t dob = head_base(rs, hi, p.sdo) + v0;
  for (int e = tid; e < K * BV; e += NTP) {
    const int kk = e / BV, c2 = e % BV;
    s.dS[kk][c2] =
        p.dfs ? p.dfs[bi * p.sdfs[0] + hi * p.sdfs[1] + kk * p.sdfs[2] + (v0 + c2) * p.sdfs[3]] : 0.f;
  }
  RNext<TIn, K> nx;
  if (nch > 0) {
    const int t0 = (nch - 1) * C;
    nx.load(p, tid, (slot0 + nch - 1) * p.H + hi, qg, kg, dob, t0, rs.T - t0);
    nx.store(s, tid, p.do_dtype);
  }
  __syncthreads();
  for (int c = nch - 1; c >= 0; --c) {
    const int64_t ri = (slot0 + c) * p.H + hi;
    if (c > 0) nx.load(p, tid, ri - p.H, qg, kg, dob, (c - 1) * C, C);
    float* const ckd = p.ckD + ri * (int64_t)K * p.V + v0;
    float* const duo = p.du + ri * (int64_t)C * p.V + v0;
    store_state<K>(tid, s.dS, ckd, p.V);
    // partial du = [scale P^T, diag(D) K] [dO; dS'] over this wave's range
    {
      f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
      split_tiles<LEN, C>(
          acc, wave * LEN, r, kq, [&](int m, int kk) { return scale * s.pm[kk][m]; },
          [&](int kk, int n) { return s.dO[kk][n]; }, [&](int m, int kk) { return s.D[m] * s.k[m][kk]; },
          [&](int kk, int n) { return s.dS[kk][n]; });
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s.part[wave][4 * kq + i][r] = acc[0][i];
        s.part[wave][16 + 4 * kq + i][r] = acc[1][i];
      }
    }
    __syncthreads();
    // du = the sum of the partial tiles, once
#pragma unroll
    for (int i = 0; i < C * BV / NTP; ++i) {
      const int e = tid + i * NTP, m = e / BV, n = e % BV;
      float x = s.part[0][m][n];
#pragma unroll
      for (int w = 1; w < NWP; ++w) x += s.part[w][m][n];
      s.du[m][n] = x;
      duo[(int64_t)m * p.V + n] = x;
    }
    __syncthreads();
    // dS <- scale Q^T diag(gam) dO + gam_C dS' - W^T du
    mmx<NTP, K, BV>(tid, [&](int m, int n, float x) { s.dS[m][n] = x + s.gC * s.dS[m][n]; },
                    seg<C>([&](int m, int kk) { return scale * s.gam[kk] * s.q[kk][m]; },
                           [&](int kk, int n) { return s.dO[kk][n]; }),
                    seg<C>([&](int m, int kk) { return -s.w[kk][m]; }, [&](int kk, int n) { return s.du[kk][n]; }));
    __syncthreads();
    if (c > 0) {
      nx.store(s, tid, p.do_dtype);
      __syncthreads();
    }
  }
  if (p.dh0 != nullptr) {
    for (int e = tid; e < K * BV; e += NTP) {
      const int kk = e / BV, c2 = e % BV;
      p.dh0[bi * p.sdh0[0] + hi * p.sdh0[1] + kk * p.sdh0[2] + (v0 + c2) * p.sdh0[3]] = s.dS[kk][c2];
    }
  }
}

template <typename TIn, int K>
__global__ __launch_bounds__(NTP) void recur_kernel(const BArgs p) {
  __shared__ FRSmem<K> sm;
  int blk = blockIdx.x;
  const bool backward = blk >= p.units;
  if (backward) blk -= p.units;
  // consecutive units (the V-slices of one head) on one XCD: they read the
  // same records
  int unit = blk;
  if (p.xcd_remap) unit = (blk & 7) * (p.units >> 3) + (blk >> 3);
  const int vs = unit % p.nv;
  const int bh = unit / p.nv;
  const int bi = bh / p.H;
  const int hi = bh % p.H;
  const RowSpan rs = row_span(p.cu, p.T, bi);
  const int64_t slot0 = p.cu ? rs.t0 / C + bi : (int64_t)bi * p.nchmax;
  if (backward) walk_backward<TIn, K>(p, sm.r, rs, bi, hi, vs * BV, slot0);
  else walk_forward<TIn, K>(p, sm.f, rs, bi, hi, vs * BV, slot0);
}

// ---------------------------------------------------------------------------
// 2b. the two recurrences for 16-bit q, k, v and dO: fp16 MFMA on hi + lo
//     operand pairs (v_mfma_f32_16x16x32_f16, lane layout in
//     gdn_tiles_f16.h).  The carried state (S or dS) lives in fp32 in the
//     accumulators of the four waves (rows 16 (w + 4 j) of K); an fp16 hi /
//     lo copy of its transpose in LDS feeds the products through it.  K^T,
//     Q^T, P^T and W^T are read from row-major LDS copies by transposing
//     reads.  Per chunk: the u (du) tiles on waves 0-1, then the state
//     update on all four waves; the inputs of the chunks ahead arrive in
//     LDS by LDS-DMA copies that waves 2-3 (and, for q, waves 0-1) issue
//     and drain themselves.
// ---------------------------------------------------------------------------

namespace w16 {

using tiles16::HP;
using tiles16::frag8;
using tiles16::frag4_t;
using tiles16::store_pair4;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// A chunk's inputs reach LDS by LDS-DMA: global_load_lds_dwordx4 (_dword)
// copies 16 (4) bytes a lane from global memory to LDS at M0 + 16 (4) lane,
// complete once the issuing wave's vmcnt has drained.  The walks' barriers
// wait for LDS accesses only, so copies issued in a chunk's first phase stay
// in flight across its other two; the issuing waves drain them before the
// chunk's last barrier.  The copies are written as inline assembly: the
// compiler then sees no LDS write in flight and adds no vmcnt wait before
// the transposing LDS reads (which it cannot tell apart from the copies'
// targets).  M0 is written here and nowhere else in these kernels.
// LDS address of a generic pointer into LDS: its low 32 bits (the LDS
// aperture sits in the high half)
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* src, void* lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_addr(lds_base))
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* src, void* lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds_addr(lds_base))
               : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ f16x4 read_tr4(const f16* a) {
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)a));
}

// Rows of W halves (W = 32, 64, 128) unpadded in LDS, each row's 16-byte
// pieces permuted: piece s of row t sits at s ^ swz<W>(t).  The 16 rows that
// a row read (frag8, 16-lane passes) takes at one piece, and the 8 rows x 2
// pieces of a pass of a transposing read (frag8_ts, 32-lane passes), then
// use every bank once.
template <int W>
__device__ __forceinline__ int swz(int t) {
  if constexpr (W == 128) return (((t >> 3) & 1) << 3) | ((t & 3) << 1) | ((t >> 2) & 1);
  else if constexpr (W == 64) return (((t >> 3) & 1) << 2) | (((t >> 1) & 1) << 1) | ((t >> 2) & 1);
  else {
    static_assert(W == 32, "rows of 32, 64 or 128 halves");
    return (((t >> 3) & 1) << 1) | ((t >> 2) & 1);
  }
}
// offset in halves of element (t, col)
template <int W>
__device__ __forceinline__ int soff(int t, int col) {
  return t * W + ((((col >> 3) ^ swz<W>(t))) << 3) + (col & 7);
}
// halves col .. col + 7 of row t
template <int W>
__device__ __forceinline__ f16x8 frag8_s(const f16* x, int t, int col) {
  return frag8(x + soff<W>(t, col));
}
// Row m0 + r of X^T, contraction indices t0 + 8 kq .. + 7, by two
// ds_read_b64_tr_b16 (lane layout as tiles16::frag8_t)
template <int W>
__device__ __forceinline__ f16x8 frag8_ts(const f16* x, int t0, int m0, int r, int kq) {
  const int t = t0 + 8 * kq + (r >> 2), col = m0 + 4 * (r & 3);
  const f16x4 lo = read_tr4(x + soff<W>(t, col)), hi = read_tr4(x + soff<W>(t + 4, col));
  return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// dO rows of a slice (BV halves) in LDS: row t at row dperm(t), bits 2 and
// 3 of t swapped, so that the rows of a 32-lane pass of a transposing read
// (t = 0..3 and 8..11, + 4 h) fill 256 contiguous bytes.
__device__ __forceinline__ int dperm(int t) { return (t & ~12) | ((t & 4) << 1) | ((t & 8) >> 1); }
// lane (r, kq) receives dO[8 kq + j][r], j = 0..7: row r of dO^T
__device__ __forceinline__ f16x8 dot_frag8(const f16* x, int r, int kq) {
  const int t = 8 * kq + (r >> 2), col = 4 * (r & 3);
  const f16x4 lo = read_tr4(x + dperm(t) * BV + col), hi = read_tr4(x + dperm(t + 4) * BV + col);
  return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Rows t0 .. t0 + C - 1 of a row-major 16-bit input (rows ld elements apart,
// row starts 16-byte aligned; rows >= nval read row nval - 1) -> rows of W
// halves swizzled by swz<W>.  The tile's C W / 512 copies (16 bytes a lane)
// are shared round robin by NW waves (this one: lw).
template <int W, int NW>
__device__ __forceinline__ void dma_rows(const uint16_t* src, int64_t ld, int nval, f16* dst, int lw, int lane) {
  constexpr int NJ = C * W / 512;
  static_assert(NJ % NW == 0, "whole copies per wave");
#pragma unroll
  for (int jj = 0; jj < NJ / NW; ++jj) {
    const int j = NW * jj + lw;
    const int pos = 512 * j + 8 * lane;  // halves
    const int t = pos / W, pc = (pos % W) / 8;
    dma16(src + min(t, nval - 1) * ld + 8 * (pc ^ swz<W>(t)), dst + 512 * j);
  }
}
// Once a wave's copies of dma_rows have landed: bf16 -> fp16, rows >= nval
// -> zero, each lane on the pieces it copied itself.
template <typename TIn, int W, int NW>
__device__ __forceinline__ void fix_rows(f16* dst, int nval, int lw, int lane) {
  constexpr int NJ = C * W / 512;
#pragma unroll
  for (int jj = 0; jj < NJ / NW; ++jj) {
    const int pos = 512 * (NW * jj + lw) + 8 * lane;
    f16x8* const a = reinterpret_cast<f16x8*>(dst + pos);
    if (pos / W >= nval) {
      *a = f16x8{};
    } else if constexpr (!std::is_same<TIn, f16>::value) {
      f16 x[8];
      InTraits<TIn>::to_op(*reinterpret_cast<const uint4*>(a), x);
      *a = f16x8{x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]};
    }
  }
}

// Rows t0 .. t0 + C - 1 of a BV-column slice of dO (rows ld elements apart,
// 4-byte aligned; rows >= nval read row nval - 1) -> rows at dperm(t): 4
// bytes a lane, C BV / 128 copies alternating between the loader waves.
__device__ __forceinline__ void dma_dot(const uint16_t* src, int64_t ld, int nval, f16* dst, int lw, int lane) {
  constexpr int NJ = C * BV / 128;
#pragma unroll
  for (int jj = 0; jj < NJ / 2; ++jj) {
    const int j = 2 * jj + lw;
    const int pos = 128 * j + 2 * lane;
    dma4(src + min(dperm(pos / BV), nval - 1) * ld + pos % BV, dst + 128 * j);
  }
}
// bf16 values times sc (a power of two: exact) -> fp16, rows >= nval -> zero
template <typename TIn>
__device__ __forceinline__ void fix_dot(f16* dst, int nval, float sc, int lw, int lane) {
  constexpr int NJ = C * BV / 128;
#pragma unroll
  for (int jj = 0; jj < NJ / 2; ++jj) {
    const int pos = 128 * (2 * jj + lw) + 2 * lane;
    uint32_t* const a = reinterpret_cast<uint32_t*>(dst + pos);
    if (dperm(pos / BV) >= nval) {
      *a = 0u;
    } else if constexpr (!std::is_same<TIn, f16>::value) {
      const uint32_t w = *a;
      const f16 lo = (f16)(bf16_bits_to_float(w & 0xffffu) * sc), hi = (f16)(bf16_bits_to_float(w >> 16) * sc);
      *a = (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
    }
  }
}

// Rows t0 .. t0 + C - 1 of a BV-column slice of v (16-byte aligned rows, as
// q, k, v are) -> rows of BV halves in order: one copy, 16 bytes a lane.
__device__ __forceinline__ void dma_v(const uint16_t* src, int64_t ld, int nval, f16* dst, int lane) {
  static_assert(C * BV == 512, "one copy");
  const int pos = 8 * lane;
  dma16(src + min(pos / BV, nval - 1) * ld + pos % BV, dst);
}
template <typename TIn>
__device__ __forceinline__ void fix_v(f16* dst, int nval, float sc, int lane) {
  const int pos = 8 * lane;
  f16x8* const a = reinterpret_cast<f16x8*>(dst + pos);
  if (pos / BV >= nval) {
    *a = f16x8{};
  } else if constexpr (!std::is_same<TIn, f16>::value) {
    f16 x[8];
    InTraits<TIn>::to_op_sc(*reinterpret_cast<const uint4*>(a), x, sc);
    *a = f16x8{x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]};
  }
}

// A chunk's inputs of the forward walk in LDS.
template <int K>
struct alignas(16) FIn {
  f16 k[C * K];               // K rows, swz<K>
  f16 th[C * C], tl[C * C];   // T diag(beta) as fp16 pairs, swz<C>
  f16 v[C * BV];              // V rows of the slice
  float gv[4][C];             // b, gam, D, {gam_C, 0 ..}
};

// The forward walk's inputs are triple-buffered (chunk c in in[c % 3]): a
// chunk's copies are issued two chunks ahead and have a whole chunk to land.
template <int K>
struct alignas(16) FMem {
  f16 sh[BV][K + HP], sl[BV][K + HP];  // S^T
  f16 yh[BV][C + HP], yl[BV][C + HP];  // (V - diag(gam) K S)^T
  f16 dh[BV][C + HP], dl[BV][C + HP];  // (diag(D) u)^T
  float uf[C][BV];                     // u rows, on their way to uu
  FIn<K> in[3];
};

// A chunk's inputs of the backward walk in LDS.
template <int K>
struct alignas(16) RIn {
  f16 q[C * K], k[C * K];     // Q, K rows, swz<K>
  f16 th[C * C], tl[C * C];   // T diag(beta), swz<C>
  f16 ph[C * C], pl[C * C];   // P, swz<C>
  f16 dot[C * BV];            // dO rows of the slice, row t at dperm(t)
  float gv[4][C];
};

template <int K>
struct alignas(16) RMem {
  f16 sh[BV][K + HP], sl[BV][K + HP];  // dS'^T
  f16 gh[BV][C + HP], gl[BV][C + HP];  // (diag(gam) dO)^T
  f16 uh[BV][C + HP], ul[BV][C + HP];  // du^T
  f16 zh[BV][C + HP], zl[BV][C + HP];  // (diag(gam) (T diag(beta))^T du)^T
  float duf[C][BV];                    // du rows, on their way to du
  RIn<K> in[2];
};

template <int K>
union Mem {
  FMem<K> f;
  RMem<K> r;
};

template <int K>
struct State {
  static constexpr int NST = (K / 16 + 3) / 4;
  f32x4 st[NST];
  // times sc (a power of two: exact)
  __device__ __forceinline__ void load(const float* src, const int64_t (&sd)[4], int bi, int hi, int v0, int wave,
                                       int r, int kq, float sc = 1.f) {
#pragma unroll
    for (int j = 0; j < NST; ++j) {
      const int m0 = 16 * (wave + 4 * j);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        st[j][i] = (src && m0 < K) ? src[bi * sd[0] + hi * sd[1] + (m0 + 4 * kq + i) * sd[2] + (v0 + r) * sd[3]] * sc
                                   : 0.f;
    }
  }
  template <int LD>
  __device__ __forceinline__ void put(f16 (*sh)[LD], f16 (*sl)[LD], int wave, int r, int kq) const {
#pragma unroll
    for (int j = 0; j < NST; ++j) {
      const int m0 = 16 * (wave + 4 * j);
      if (m0 < K) {
        const float x[4] = {st[j][0], st[j][1], st[j][2], st[j][3]};
        store_pair4(&sh[r][m0 + 4 * kq], &sl[r][m0 + 4 * kq], x);
      }
    }
  }
};

// The state's fp16 values -> rows of the [V][K] chunk-state array (row =
// state column), 16 bytes a lane (NT lanes).  They are the hi parts of the walk's
// S^T pair copy (x rounded to nearest), copied as they are.
template <int K, int NT, int LD>
__device__ __forceinline__ void copy_state_rows(const f16 (*sh)[LD], f16* dst, int tid) {
  constexpr int NV = BV * K / 8;
#pragma unroll
  for (int i = 0; i < (NV + NT - 1) / NT; ++i) {
    const int e = tid + i * NT;
    if (NV % NT == 0 || e < NV)
      *reinterpret_cast<f16x8*>(dst + (int64_t)(e / (K / 8)) * K + 8 * (e % (K / 8))) =
          *reinterpret_cast<const f16x8*>(&sh[e / (K / 8)][8 * (e % (K / 8))]);
  }
}

// Forward walk: S at each chunk start -> ckS (fp16), u -> uu.  For bf16
// inputs the walk runs on v and h0 shifted into fp16's range
// (slice_range_scale: both outputs are linear in them) and shifts u back;
// ckS stays in the shifted units, and the factor that takes it back goes to
// scl[unit].  Waves 2 and 3 (the loaders) carry every global access of the
// loop, chunks alternating between them: in chunk c wave 2 + c % 2 issues
// the copies of chunk c + 2 and stores chunk c's state rows and u rows,
// while the other waits for the copies of chunk c + 1 it issued a chunk
// earlier (its only memory operations in flight).  Waves 0 and 1 hold the
// chain's products (Y, u).
template <typename TIn, int K>
__device__ __forceinline__ void walk_forward16(const BArgs& p, FMem<K>& s, const RowSpan& rs, int bi, int hi,
                                               int v0, int64_t slot0) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, kq = lane >> 4;
  const int nch = (rs.T + C - 1) / C;
  const TIn* const kg = static_cast<const TIn*>(p.k) + head_base(rs, hi, p.sk);
  const TIn* const vg = static_cast<const TIn*>(p.v) + head_base(rs, hi, p.sv) + v0;
  const RangeScale rsc = slice_range_scale<TIn>(
      reinterpret_cast<const char*>(vg), p.sv[1] * (int64_t)sizeof(TIn), rs.T, BV,
      p.h0 ? p.h0 + bi * p.sh0[0] + hi * p.sh0[1] + v0 * p.sh0[3] : nullptr, p.sh0[2], p.sh0[3], K, 1.f);
  if (tid == 0) p.scl[((int64_t)bi * p.H + hi) * p.nv + v0 / BV] = rsc.fs;
  const bool loader = wave >= 2;
  const int lw = wave - 2;
  // a loader: chunk cn's inputs -> in[b]
  auto fetch = [&](int cn, int b) __attribute__((always_inline)) {
    FIn<K>& d = s.in[b];
    const int64_t ri = (slot0 + cn) * p.H + hi;
    const int nval = min(C, rs.T - cn * C);
    const uint16_t* const rh = reinterpret_cast<const uint16_t*>(p.r16 + ri * (int64_t)Rec16::SIZE);
    dma_rows<K, 1>(reinterpret_cast<const uint16_t*>(kg) + (int64_t)cn * C * p.sk[1], p.sk[1], nval, d.k, 0, lane);
    dma_rows<C, 1>(rh + Rec16::TBH, C, C, d.th, 0, lane);
    dma_rows<C, 1>(rh + Rec16::TBL, C, C, d.tl, 0, lane);
    dma_v(reinterpret_cast<const uint16_t*>(vg) + (int64_t)cn * C * p.sv[1], p.sv[1], nval, d.v, lane);
    if (lane < C) dma16(p.rec + ri * (int64_t)RecT::SIZE + RecT::G + 4 * lane, &d.gv[0][0]);
  };
  // the loader that fetched chunk cn, before the barrier that publishes it
  auto settle = [&](int cn, int b) __attribute__((always_inline)) {
    wait_dma();
    const int nval = min(C, rs.T - cn * C);
    if (!std::is_same<TIn, f16>::value || nval < C) {
      fix_rows<TIn, K, 1>(s.in[b].k, nval, 0, lane);
      fix_v<TIn>(s.in[b].v, nval, rsc.v, lane);
    }
  };
  State<K> S;
  S.load(p.h0, p.sh0, bi, hi, v0, wave, r, kq, rsc.v);
  S.put(s.sh, s.sl, wave, r, kq);
  if (loader && lw < nch) {
    fetch(lw, lw);
    if (lw == 0) settle(0, 0);
  }
  bar();
  for (int c = 0, b = 0; c < nch; ++c, b = b == 2 ? 0 : b + 1) {
    const int64_t ri = (slot0 + c) * p.H + hi;
    FIn<K>& in = s.in[b];
    const int b1 = b == 2 ? 0 : b + 1, b2 = b1 == 2 ? 0 : b1 + 1;
    const bool issuer = loader && lw == (c & 1);
    if (!loader) {
      // Y = V - diag(gam) K S for rows 16 w .. (k exact in fp16), as Y^T pairs
      const int um0 = 16 * wave;
      f32x4 ak = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < K; kb += 32) {
        const f16x8 kf = frag8_s<K>(in.k, um0 + r, kb + 8 * kq);
        ak = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, frag8(&s.sh[r][kb + 8 * kq]), ak, 0, 0, 0);
        ak = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, frag8(&s.sl[r][kb + 8 * kq]), ak, 0, 0, 0);
      }
      const int t = um0 + 4 * kq;
      const f16x4 vv = frag4_t(reinterpret_cast<const f16 (*)[BV]>(in.v), um0, 0, r, kq);
      const float y[4] = {(float)vv[0] - in.gv[1][t] * ak[0], (float)vv[1] - in.gv[1][t + 1] * ak[1],
                          (float)vv[2] - in.gv[1][t + 2] * ak[2], (float)vv[3] - in.gv[1][t + 3] * ak[3]};
      store_pair4(&s.yh[r][t], &s.yl[r][t], y);
    } else if (issuer && c + 2 < nch) {
      fetch(c + 2, b2);
    }
    bar();
    if (!loader) {
      // u = T diag(beta) Y, rows 16 w .. (W S = T diag(beta) diag(gam) K S)
      const int um0 = 16 * wave;
      f32x4 au = {0.f, 0.f, 0.f, 0.f};
      const f16x8 th = frag8_s<C>(in.th, um0 + r, 8 * kq), yh = frag8(&s.yh[r][8 * kq]);
      au = __builtin_amdgcn_mfma_f32_16x16x32_f16(th, yh, au, 0, 0, 0);
      au = __builtin_amdgcn_mfma_f32_16x16x32_f16(th, frag8(&s.yl[r][8 * kq]), au, 0, 0, 0);
      au = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag8_s<C>(in.tl, um0 + r, 8 * kq), yh, au, 0, 0, 0);
      const int t = um0 + 4 * kq;
      float du[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        du[i] = in.gv[2][t + i] * au[i];
        s.uf[t + i][r] = au[i] * rsc.fs;
      }
      store_pair4(&s.dh[r][t], &s.dl[r][t], du);
    } else if (issuer) {
      copy_state_rows<K, 64>(s.sh, reinterpret_cast<f16*>(p.ckS) + (ri * p.V + v0) * (int64_t)K, lane);
    }
    bar();
    // S <- gam_C S + K^T diag(D) u
#pragma unroll
    for (int j = 0; j < State<K>::NST; ++j) {
      const int m0 = 16 * (wave + 4 * j);
      if (m0 < K) {
        const f16x8 kt = frag8_ts<K>(in.k, 0, m0, r, kq);
        f32x4 a = {0.f, 0.f, 0.f, 0.f};
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kt, frag8(&s.dh[r][8 * kq]), a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kt, frag8(&s.dl[r][8 * kq]), a, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) S.st[j][i] = in.gv[3][0] * S.st[j][i] + a[i];
      }
    }
    S.put(s.sh, s.sl, wave, r, kq);
    if (issuer) {
      // u rows -> uu: 16 bytes a lane
      static_assert(C * BV % (4 * 64) == 0, "whole u pieces per lane");
#pragma unroll
      for (int i = 0; i < C * BV / (4 * 64); ++i) {
        const int e = lane + 64 * i, row = e / (BV / 4), c4 = 4 * (e % (BV / 4));
        *reinterpret_cast<f32x4*>(p.uu + (ri * C + row) * (int64_t)p.V + v0 + c4) =
            *reinterpret_cast<const f32x4*>(&s.uf[row][c4]);
      }
    } else if (loader && c + 1 < nch) {
      settle(c + 1, b1);
    }
    bar();
  }
  wait_dma();
}

// Backward walk: dS' of each chunk -> ckD (fp16), du -> du, at the end dh0.
// For bf16 inputs the walk runs on dO and d_final_state shifted into fp16's
// range (every output of the walk is linear in them) and shifts du and dh0
// back: small gradients keep their hi / lo precision.  ckD stays in the
// shifted units; the factor that takes it back goes to scl[units + unit].
// Waves 2 and 3 (the loaders) copy the previous chunk's inputs but its q
// rows and store the chunk's dS' rows and du rows; waves 0 and 1 hold the
// chain's products (du, z) and copy the q rows once their du is done.
template <typename TIn, int K>
__device__ __forceinline__ void walk_backward16(const BArgs& p, RMem<K>& s, const RowSpan& rs, int bi, int hi,
                                                int v0, int64_t slot0) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, kq = lane >> 4;
  const int nch = (rs.T + C - 1) / C;
  const float scale = p.scale;
  const TIn* const qg = static_cast<const TIn*>(p.q) + head_base(rs, hi, p.sq);
  const TIn* const kg = static_cast<const TIn*>(p.k) + head_base(rs, hi, p.sk);
  const TIn* const dg = static_cast<const TIn*>(p.d_o) + head_base(rs, hi, p.sdo) + v0;
  const RangeScale rsd = slice_range_scale<TIn>(
      reinterpret_cast<const char*>(dg), p.sdo[1] * (int64_t)sizeof(TIn), rs.T, BV,
      p.dfs ? p.dfs + bi * p.sdfs[0] + hi * p.sdfs[1] + v0 * p.sdfs[3] : nullptr, p.sdfs[2], p.sdfs[3], K, 1.f);
  if (tid == 0) p.scl[p.units + ((int64_t)bi * p.H + hi) * p.nv + v0 / BV] = rsd.fs;
  const bool loader = wave >= 2;
  const int lw = wave - 2, ll = tid - 128;
  // chunk cn's inputs -> in[cn & 1]: q rows from waves 0 and 1 (issued at
  // the end of their first phase, where they wait for the loaders anyway),
  // the rest from the loaders
  auto fetch = [&](int cn) __attribute__((always_inline)) {
    RIn<K>& d = s.in[cn & 1];
    const int nval = min(C, rs.T - cn * C);
    if (!loader) {
      dma_rows<K, 2>(reinterpret_cast<const uint16_t*>(qg) + (int64_t)cn * C * p.sq[1], p.sq[1], nval, d.q, wave,
                     lane);
      return;
    }
    const int64_t ri = (slot0 + cn) * p.H + hi;
    const uint16_t* const rh = reinterpret_cast<const uint16_t*>(p.r16 + ri * (int64_t)Rec16::SIZE);
    dma_rows<K, 2>(reinterpret_cast<const uint16_t*>(kg) + (int64_t)cn * C * p.sk[1], p.sk[1], nval, d.k, lw, lane);
    dma_rows<C, 2>(rh + Rec16::TBH, C, C, d.th, lw, lane);
    dma_rows<C, 2>(rh + Rec16::TBL, C, C, d.tl, lw, lane);
    dma_rows<C, 2>(rh + Rec16::PH, C, C, d.ph, lw, lane);
    dma_rows<C, 2>(rh + Rec16::PL, C, C, d.pl, lw, lane);
    dma_dot(reinterpret_cast<const uint16_t*>(dg) + (int64_t)cn * C * p.sdo[1], p.sdo[1], nval, d.dot, lw, lane);
    if (lw == 0 && lane < C) dma16(p.rec + ri * (int64_t)RecT::SIZE + RecT::G + 4 * lane, &d.gv[0][0]);
  };
  // every wave, before the barrier that publishes chunk cn: its own copies
  auto settle = [&](int cn) __attribute__((always_inline)) {
    wait_dma();
    const int nval = min(C, rs.T - cn * C);
    if (!std::is_same<TIn, f16>::value || nval < C) {
      RIn<K>& d = s.in[cn & 1];
      if (!loader) {
        fix_rows<TIn, K, 2>(d.q, nval, wave, lane);
      } else {
        fix_rows<TIn, K, 2>(d.k, nval, lw, lane);
        fix_dot<TIn>(d.dot, nval, rsd.v, lw, lane);
      }
    }
  };
  State<K> S;
  S.load(p.dfs, p.sdfs, bi, hi, v0, wave, r, kq, rsd.v);
  S.put(s.sh, s.sl, wave, r, kq);
  if (nch > 0) {
    fetch(nch - 1);
    settle(nch - 1);
  }
  bar();
  for (int c = nch - 1; c >= 0; --c) {
    const int64_t ri = (slot0 + c) * p.H + hi;
    RIn<K>& in = s.in[c & 1];
    if (!loader) {
      // du = scale P^T dO + diag(D) K dS', rows 16 w ..
      const int um0 = 16 * wave;
      f32x4 a1 = {0.f, 0.f, 0.f, 0.f}, a2 = {0.f, 0.f, 0.f, 0.f};
      const f16x8 df = dot_frag8(in.dot, r, kq);
      a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag8_ts<C>(in.ph, 0, um0, r, kq), df, a1, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(frag8_ts<C>(in.pl, 0, um0, r, kq), df, a1, 0, 0, 0);
#pragma unroll
      for (int kb = 0; kb < K; kb += 32) {
        const f16x8 kf = frag8_s<K>(in.k, um0 + r, kb + 8 * kq);
        a2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, frag8(&s.sh[r][kb + 8 * kq]), a2, 0, 0, 0);
        a2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, frag8(&s.sl[r][kb + 8 * kq]), a2, 0, 0, 0);
      }
      const int t = um0 + 4 * kq;
      float du[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        du[i] = scale * a1[i] + in.gv[2][t + i] * a2[i];
        s.duf[t + i][r] = du[i] * rsd.fs;
      }
      store_pair4(&s.uh[r][t], &s.ul[r][t], du);
      if (c >= 1) fetch(c - 1);
    } else {
      // the previous chunk's copies first: they have until the chunk's end
      if (c >= 1) fetch(c - 1);
      // (diag(gam) dO)^T as pairs: lane (r, kq) of loader wave lw -> column
      // r, rows t4 .. t4 + 3 (a 32-lane pass reads rows 0..3, 8..11 + 16 lw)
      const int t4 = 16 * lw + ((kq & 1) << 3) + ((kq & 2) << 1);
      const f16x4 dv = read_tr4(in.dot + dperm(t4 + (r >> 2)) * BV + 4 * (r & 3));
      const float x[4] = {in.gv[1][t4] * (float)dv[0], in.gv[1][t4 + 1] * (float)dv[1],
                          in.gv[1][t4 + 2] * (float)dv[2], in.gv[1][t4 + 3] * (float)dv[3]};
      store_pair4(&s.gh[r][t4], &s.gl[r][t4], x);
      copy_state_rows<K, 128>(s.sh, reinterpret_cast<f16*>(p.ckD) + (ri * p.V + v0) * (int64_t)K, ll);
    }
    bar();
    // W^T du = K^T diag(beta gam) T^T du = K^T (diag(gam) (T diag(beta))^T du):
    // z on waves 0-1 (rows 16 w .. of z, T diag(beta) transposed by the
    // reads) while waves 2-3 form their Q^T diag(gam) dO term
    f32x4 aq[State<K>::NST];
    auto q_term = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < State<K>::NST; ++j) {
        const int m0 = 16 * (wave + 4 * j);
        aq[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (m0 < K) {
          const f16x8 qt = frag8_ts<K>(in.q, 0, m0, r, kq);
          aq[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qt, frag8(&s.gh[r][8 * kq]), aq[j], 0, 0, 0);
          aq[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qt, frag8(&s.gl[r][8 * kq]), aq[j], 0, 0, 0);
        }
      }
    };
    if (!loader) {
      const int um0 = 16 * wave;
      const f16x8 tth = frag8_ts<C>(in.th, 0, um0, r, kq), ttl = frag8_ts<C>(in.tl, 0, um0, r, kq);
      const f16x8 uh = frag8(&s.uh[r][8 * kq]);
      f32x4 az = {0.f, 0.f, 0.f, 0.f};
      az = __builtin_amdgcn_mfma_f32_16x16x32_f16(tth, uh, az, 0, 0, 0);
      az = __builtin_amdgcn_mfma_f32_16x16x32_f16(tth, frag8(&s.ul[r][8 * kq]), az, 0, 0, 0);
      az = __builtin_amdgcn_mfma_f32_16x16x32_f16(ttl, uh, az, 0, 0, 0);
      const int t = um0 + 4 * kq;
      const float z[4] = {in.gv[1][t] * az[0], in.gv[1][t + 1] * az[1], in.gv[1][t + 2] * az[2],
                          in.gv[1][t + 3] * az[3]};
      store_pair4(&s.zh[r][t], &s.zl[r][t], z);
    } else {
      q_term();
      // du rows -> du: 16 bytes a loader lane
      static_assert(C * BV == 4 * 128, "four du entries per loader lane");
      const int row = ll / (BV / 4), c4 = 4 * (ll % (BV / 4));
      *reinterpret_cast<f32x4*>(p.du + (ri * C + row) * (int64_t)p.V + v0 + c4) =
          *reinterpret_cast<const f32x4*>(&s.duf[row][c4]);
    }
    bar();
    if (!loader) q_term();
    // dS <- scale Q^T diag(gam) dO + gam_C dS' - K^T z
#pragma unroll
    for (int j = 0; j < State<K>::NST; ++j) {
      const int m0 = 16 * (wave + 4 * j);
      if (m0 < K) {
        const f16x8 kt = frag8_ts<K>(in.k, 0, m0, r, kq);
        f32x4 b = {0.f, 0.f, 0.f, 0.f};
        b = __builtin_amdgcn_mfma_f32_16x16x32_f16(kt, frag8(&s.zh[r][8 * kq]), b, 0, 0, 0);
        b = __builtin_amdgcn_mfma_f32_16x16x32_f16(kt, frag8(&s.zl[r][8 * kq]), b, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) S.st[j][i] = scale * aq[j][i] + in.gv[3][0] * S.st[j][i] - b[i];
      }
    }
    S.put(s.sh, s.sl, wave, r, kq);
    if (c >= 1) settle(c - 1);
    bar();
  }
  wait_dma();
  if (p.dh0 != nullptr) {
#pragma unroll
    for (int j = 0; j < State<K>::NST; ++j) {
      const int m0 = 16 * (wave + 4 * j);
      if (m0 < K) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          p.dh0[bi * p.sdh0[0] + hi * p.sdh0[1] + (m0 + 4 * kq + i) * p.sdh0[2] + (v0 + r) * p.sdh0[3]] =
              S.st[j][i] * rsd.fs;
      }
    }
  }
}

}  // namespace w16

template <typename TIn, int K>
__global__ __launch_bounds__(NTP) void recur16_kernel(const BArgs p) {
  __shared__ w16::Mem<K> sm;
  int blk = blockIdx.x;
  const bool backward = blk >= p.units;
  if (backward) blk -= p.units;
  int unit = blk;
  if (p.xcd_remap) unit = (blk & 7) * (p.units >> 3) + (blk >> 3);
  const int vs = unit % p.nv;
  const int bh = unit / p.nv;
  const int bi = bh / p.H;
  const int hi = bh % p.H;
  const RowSpan rs = row_span(p.cu, p.T, bi);
  const int64_t slot0 = p.cu ? rs.t0 / C + bi : (int64_t)bi * p.nchmax;
  if (backward) w16::walk_backward16<TIn, K>(p, sm.r, rs, bi, hi, vs * BV, slot0);
  else w16::walk_forward16<TIn, K>(p, sm.f, rs, bi, hi, vs * BV, slot0);
}

// ---------------------------------------------------------------------------
// 3. every gradient of a chunk
// ---------------------------------------------------------------------------

template <int K, int VS>
struct alignas(16) GSmem {
  // SD = VS + 4: rows of the V-step tiles are read 16 bytes per lane, lane
  // (r, kq) at row r, columns 4 kq .. 4 kq + 3 of a 16-column group; a row
  // stride of 4 (mod 32) words makes each 8-lane group's reads conflict-free.
  // KD = K + 4: accumulator-layout accesses (lane (r, kq) at row 4 kq + i,
  // column r) fall in 64 different banks, and rows are 16-byte aligned.
  static constexpr int KD = K + 4, CD = C + 1, SD = VS + 4;
  float q[C][KD], k[C][KD];
  float dw[C][KD];   // dW = -du S^T
  float dwt[C][KD];  // dW~ = T^T dW
  float t[C][CD], pm[C][CD], kk[C][CD], m[C][CD];
  float y[C][CD];    // dQK = M o (scale dO u^T)
  float yp[C][CD];   // dQK o Q K^T = scale (dO u^T) o P
  float dt[C][CD];   // dT, then dA
  float z[C][CD];    // T^T dT, then dKK
  // The V step's tiles: fp32 (w), or for fp16 inputs with fp16 states
  // MFMA operand rows in fp16 (h: v, dO and the states exact, u and du as
  // hi + lo pairs; HD = VS + 16 halves, 16-byte aligned rows).
  static constexpr int HD = VS + 16;
  union {
    struct {
      float v[C][SD], dO[C][SD], u[C][SD], du[C][SD];
      union {
        struct {
          float S[K][SD], dS[K][SD];  // fp32 states
        } f;
        struct {
          // fp16 states of the 16-bit walks, as stored; K + 16 halves (8
          // words past a multiple of 64) puts the 8-byte transposed reads
          // of 32 lanes (rows 4 kq + r / 4, columns 4 (r % 4)) in 64
          // different banks
          f16 ST[VS][K + 16], dST[VS][K + 16];
        } h;
      } st;
    } w;
    struct {
      f16 v[C][HD], dO[C][HD], uh[C][HD], ul[C][HD], dh[C][HD], dl[C][HD];
      f16 ST[VS][K + 8], dST[VS][K + 8];  // S^T, dS'^T rows (as stored)
    } h;
    // after the walk (fp16 inputs): operands of the dq / dk products, q and
    // k exact in fp16, dQK and dKK + dKK^T as hi + lo pairs, all row-major
    // (transposed operands are read with ds_read_b64_tr_b16)
    struct {
      f16 q[C][K + 8], k[C][K + 8];
      f16 dwh[C][K + 8], dwl[C][K + 8];  // dW
      f16 yh[C][C + 8], yl[C][C + 8];    // dQK
      f16 zh[C][C + 8], zl[C][C + 8];    // Z = T^T dT, later dKK + dKK^T
      f16 th[C][C + 8], tl[C][C + 8];    // T
      f16 dth[C][C + 8], dtl[C][C + 8];  // dT
    } x;
  };
  float b[C], gam[C], D[C], bt[C];
  float rq[K / 16][C], rk[K / 16][C], rw[K / 16][C];  // row partials, one row per 16-column tile
  float vu[VS / 16][C];  // v.dU~ row partials, one row per 16-column tile
  float kw[C], dgam[C], dD[C], db[C], dbt[C];
  float scs[VS], scd[VS];  // the V step's state scales per state column (16-bit walks)
  float red[NTG / 64];
  float gC, dgC;
};

// VS: V columns per step of the V walk (32, or 16 when V is an odd
// multiple of 16).  ST16: ckS and ckD hold fp16 in the walks' shifted units
// (the 16-bit walks), scaled back per 16-column slice by scl when staged.
// NVS: the number of V steps when fixed at compile time (V = 128 or 64;
// 0: V / VS at run time), so that the walk unrolls into straight-line code
// whose waits cover exactly the step being staged.
template <typename TIn, int K, int VS, bool ST16, int NVS>
__global__ __launch_bounds__(NTG) void grad_kernel(const BArgs p) {
  using R = typename std::conditional<ST16, RecT, Rec<K>>::type;
  constexpr int RL = NTG / C;
  // fp16 inputs with fp16 states (no range shift): the V walk's products on
  // v_mfma_f32_16x16x32_f16, one 32-column step per product
  constexpr bool F16W = ST16 && std::is_same<TIn, f16>::value && VS == 32;
  __shared__ GSmem<K, VS> s;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, kq = lane >> 4;
  const int64_t slot = blockIdx.x / p.H;
  const int hi = blockIdx.x % p.H;
  RowSpan rs;
  int c, seq;
  if (!slot_chunk<C>(p, slot, rs, c, seq)) return;
  const int t0 = c * C, nval = min(C, rs.T - t0);
  const float scale = p.scale;
  const int64_t ri = slot * p.H + hi;
  const float* const rec = p.rec + ri * R::SIZE;
  using TS = typename std::conditional<ST16, f16, float>::type;
  const TS* const cks = reinterpret_cast<const TS*>(p.ckS) + ri * (int64_t)K * p.V;
  const TS* const ckd = reinterpret_cast<const TS*>(p.ckD) + ri * (int64_t)K * p.V;
  // the state scales of this head's 16-column walk slices
  const float* const sclS = ST16 ? p.scl + ((int64_t)seq * p.H + hi) * p.nv : nullptr;
  const float* const sclD = ST16 ? sclS + p.units : nullptr;
  const float* const uu = p.uu + ri * (int64_t)C * p.V;
  const float* const dug = p.du + ri * (int64_t)C * p.V;
  const int64_t qb = head_base(rs, hi, p.sq) + (int64_t)t0 * p.sq[1];
  const int64_t kb = head_base(rs, hi, p.sk) + (int64_t)t0 * p.sk[1];
  const int64_t vb = head_base(rs, hi, p.sv) + (int64_t)t0 * p.sv[1];
  const int64_t dob = head_base(rs, hi, p.sdo) + (int64_t)t0 * p.sdo[1];
  const int64_t dvb = head_base(rs, hi, p.sdv) + (int64_t)t0 * p.sdv[1];
  const int64_t dqb = head_base(rs, hi, p.sdq) + (int64_t)t0 * p.sdq[1];
  const int64_t dkb = head_base(rs, hi, p.sdk) + (int64_t)t0 * p.sdk[1];

  // ---- q, k, beta and the record: loads issued here, stored to LDS with
  // the first V step's rows (one wait for both)
  RowLoad<TIn, C, K, NTG> lq, lk;
  RowLoad<float, C, C, NTG> lt, lp, lkk;
  lq.load(tid, static_cast<const TIn*>(p.q) + qb, p.sq[1], nval);
  lk.load(tid, static_cast<const TIn*>(p.k) + kb, p.sk[1], nval);
  lt.load(tid, rec + R::T, C, C);
  if constexpr (!ST16) {
    lp.load(tid, rec + R::PM, C, C);
    lkk.load(tid, rec + R::KK, C, C);
  }
  const float gate = tid < 4 * C ? rec[R::G + tid] : 0.f;
  const uint32_t bvb =
      tid < nval ? load_bits(p.beta, head_base(rs, hi, p.sb) + (int64_t)(t0 + tid) * p.sb[1], p.beta_dtype) : 0u;

  // ---- walk V in VS-column steps.  The C x K products (dW, dO S^T,
  // u dS'^T) accumulate in registers: wave w owns tiles w + 8 i of the
  // (C/16) x (K/16) tiles.
  constexpr int NCT = K / 16, NTA = (C / 16) * NCT, NPW = (NTA + 7) / 8;
  int am0[NPW], an0[NPW], ana = 0;
#pragma unroll
  for (int i = 0; i < NPW; ++i) {
    const int j = wave + 8 * i;
    am0[i] = j < NTA ? (j / NCT) * 16 : 0;
    an0[i] = j < NTA ? (j % NCT) * 16 : 0;
    if (j < NTA) ana = i + 1;
  }
  f32x4 accW[NPW], accQ[NPW], accK[NPW];
#pragma unroll
  for (int i = 0; i < NPW; ++i) {
    accW[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    accQ[i] = accW[i];
    accK[i] = accW[i];
  }
  // one C x C tile per wave: dO u^T (waves 0-3) or du (beta V)^T (waves 4-7)
  const int cm0[1] = {((wave & 3) >> 1) * 16}, cn0[1] = {(wave & 1) * 16};
  f32x4 accC[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
  // dU~ = T^T du of the step: waves 4 .. 4 + NDU - 1, one 16 x 16 tile each
  constexpr int NDU = (C / 16) * (VS / 16);
  const bool du_wave = wave >= 4 && wave < 4 + NDU;
  const int um0[1] = {((wave - 4) / (VS / 16)) * 16}, un0[1] = {((wave - 4) % (VS / 16)) * 16};
  float vu_acc[4] = {0.f, 0.f, 0.f, 0.f};
  float dgc_acc = 0.f;

  const int nvs = NVS > 0 ? NVS : p.V / VS;
  constexpr int NDO = C * VS / NTG;
  static_assert(C * VS % NTG == 0, "dO elements per thread");
  // One V step's rows in registers.  Two of them alternate, so that the
  // loads of a step are issued two steps before it (each has a whole step's
  // products to arrive).
  // Every load of a step is unconditional (rows past the chunk's end read
  // its last row again and are zeroed when stored), so that staging one
  // step waits only for that step's loads.  With the 16-bit walks dO has
  // q's dtype and 4-byte aligned rows: one element pair per thread.
  constexpr int NDP = C * VS / 2;  // dO element pairs of a step (VS = 16: waves 0-3 only)
  static_assert(!ST16 || NDP == NTG || NDP == NTG / 2, "at most one dO pair per thread");
  // states: fp32 [K][V] rows, or fp16 [V][K] rows from the 16-bit walks
  using SLoad = typename std::conditional<ST16, RowLoad<f16, VS, K, NTG>, RowLoad<float, K, VS, NTG>>::type;
  struct StepRows {
    RowLoad<TIn, C, VS, NTG> lv;
    RowLoad<float, C, VS, NTG> lu, ldu;
    SLoad lS, ldS;
    float scS[2], scD[2];
    uint32_t rdo[NDO];
  };
  auto load_step = [&](StepRows& x, int vsi) __attribute__((always_inline)) {
    const int v0 = vsi * VS;
    x.lv.load_clamped(tid, static_cast<const TIn*>(p.v) + vb + v0, p.sv[1], nval);
    x.lu.load_clamped(tid, uu + v0, p.V, C);
    x.ldu.load_clamped(tid, dug + v0, p.V, C);
    if constexpr (ST16) {
      x.lS.load_clamped(tid, cks + (int64_t)v0 * K, K, VS);
      x.ldS.load_clamped(tid, ckd + (int64_t)v0 * K, K, VS);
    } else {
      x.lS.load_clamped(tid, cks + v0, p.V, K);
      x.ldS.load_clamped(tid, ckd + v0, p.V, K);
    }
    x.scS[0] = x.scS[1] = x.scD[0] = x.scD[1] = 1.f;
    if constexpr (ST16) {
#pragma unroll
      for (int j = 0; j < VS / 16; ++j) {
        x.scS[j] = sclS[v0 / 16 + j];
        x.scD[j] = sclD[v0 / 16 + j];
      }
      const int t = tid / (VS / 2), c2 = 2 * (tid % (VS / 2));
      if (NDP == NTG || tid < NDP)
        x.rdo[0] = *reinterpret_cast<const uint32_t*>(static_cast<const TIn*>(p.d_o) + dob +
                                                      (int64_t)min(t, nval - 1) * p.sdo[1] + v0 + c2);
    } else {
#pragma unroll
      for (int i = 0; i < NDO; ++i) {
        const int e = tid + i * NTG, t = e / VS, c2 = e % VS;
        x.rdo[i] = t < nval ? load_bits(p.d_o, dob + (int64_t)t * p.sdo[1] + v0 + c2, p.do_dtype) : 0u;
      }
    }
  };
  auto store_step = [&](const StepRows& x) __attribute__((always_inline)) {
    if constexpr (F16W) {
      x.lv.store_raw(tid, s.h.v, nval);
      x.lu.store_pairs(tid, s.h.uh, s.h.ul);
      x.ldu.store_pairs(tid, s.h.dh, s.h.dl);
      x.lS.store_raw(tid, s.h.ST);
      x.ldS.store_raw(tid, s.h.dST);
      const int t = tid / (VS / 2), c2 = 2 * (tid % (VS / 2));
      if (NDP == NTG || tid < NDP) *reinterpret_cast<uint32_t*>(&s.h.dO[t][c2]) = t < nval ? x.rdo[0] : 0u;
      return;
    }
    x.lv.store_masked(tid, s.w.v, nval);
    x.lu.store(tid, s.w.u);
    x.ldu.store(tid, s.w.du);
    if constexpr (ST16) {
      // [V][K] fp16 rows as they are; the products read them transposed and
      // scale them back per 16-column slice
      x.lS.store_raw(tid, s.w.st.h.ST);
      x.ldS.store_raw(tid, s.w.st.h.dST);
      {
        // every thread writes its column's scales (the same value as the
        // other threads of the column): the scale loads are consumed on
        // every lane, so they stay where they were issued, a step ahead
        // (constant indices into the register arrays: a variable index
        // would put the step's rows in scratch memory)
        const int v = (tid / (K / 8)) % VS;
        s.scs[v] = v < 16 ? x.scS[0] : x.scS[VS / 16 - 1];
        s.scd[v] = v < 16 ? x.scD[0] : x.scD[VS / 16 - 1];
      }
      const int t = tid / (VS / 2), c2 = 2 * (tid % (VS / 2));
      if (NDP == NTG || tid < NDP) {
        // dO has q's dtype here: a compile-time conversion
        constexpr int dt = std::is_same<TIn, f16>::value ? GDN_DTYPE_F16 : GDN_DTYPE_BF16;
        const bool ok = t < nval;
        s.w.dO[t][c2] = ok ? bits_to_float(x.rdo[0] & 0xffffu, dt) : 0.f;
        s.w.dO[t][c2 + 1] = ok ? bits_to_float(x.rdo[0] >> 16, dt) : 0.f;
      }
    } else {
      x.lS.store(tid, s.w.st.f.S);
      x.ldS.store(tid, s.w.st.f.dS);
#pragma unroll
      for (int i = 0; i < NDO; ++i) {
        const int e = tid + i * NTG;
        s.w.dO[e / VS][e % VS] = bits_to_float(x.rdo[i], p.do_dtype);
      }
    }
  };
  StepRows ra, rb;
  load_step(ra, 0);
  lq.store(tid, s.q);
  lk.store(tid, s.k);
  lt.store(tid, s.t);
  if constexpr (!ST16) {
    lp.store(tid, s.pm);
    lkk.store(tid, s.kk);
  }
  if (tid < C) {
    s.b[tid] = gate;
    s.bt[tid] = bits_to_float(bvb, p.beta_dtype);
  } else if (tid < 2 * C) {
    s.gam[tid - C] = gate;
  } else if (tid < 3 * C) {
    s.D[tid - 2 * C] = gate;
  } else if (tid == 3 * C) {
    s.gC = gate;
  }
  store_step(ra);
  if (nvs > 1) load_step(rb, 1);
  __syncthreads();
  for (int e = tid; e < C * C; e += NTG) {
    const int t = e / C, j = e % C;
    s.m[t][j] = j <= t ? expf(s.b[t] - s.b[j]) : 0.f;
  }
  if constexpr (ST16 && !F16W) {
    // K K^T (waves 0-3) and P = M o Q K^T (waves 4-7) from the 16-bit q
    // and k rows (the 16-bit prep does not store them): one 16 x 16 tile
    // per wave, the products exact and the sums in fp32 as in the prep
    // (fp16 inputs form them after the V walk instead)
    const int mt = (wave >> 1) & 1, nt = wave & 1;
    constexpr int KD = GSmem<K, VS>::KD;
    const float* const arow = (wave < 4 ? &s.k[0][0] : &s.q[0][0]) + (16 * mt + r) * KD + 8 * kq;
    const float* const brow = &s.k[0][0] + (16 * nt + r) * KD + 8 * kq;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < K; kb += 32) acc = mma16<TIn>(pack16<TIn>(arow + kb), pack16<TIn>(brow + kb), acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * mt + 4 * kq + i, j = 16 * nt + r;
      if (wave < 4) s.kk[t][j] = acc[i];
      else s.pm[t][j] = j <= t ? expf(s.b[t] - s.b[j]) * acc[i] : 0.f;
    }
  }
  // step vsi: `cur` holds step vsi + 1's rows (loaded a step ago), `nxt`
  // receives step vsi + 2's
  // this thread's part of <S, dS'> over the step's fp16 state rows ([V][K]
  // as stored): 8 consecutive keys of state column tid / (K / 8), times the
  // column's two scales
  auto state_dot = [&](const auto& st, const auto& dst, float fs, float fd) __attribute__((always_inline)) {
    static_assert(VS * K / 8 <= NTG, "one 8-key piece per thread at most");
    float x = 0.f;
    const int v = tid / (K / 8), k0 = 8 * (tid % (K / 8));
    if (VS * K / 8 == NTG || tid < VS * K / 8) {
      const f16x8 a = *reinterpret_cast<const f16x8*>(&st[v][k0]);
      const f16x8 b = *reinterpret_cast<const f16x8*>(&dst[v][k0]);
#pragma unroll
      for (int j = 0; j < 8; ++j) x = __builtin_fmaf((float)a[j], (float)b[j], x);
    }
    return x * (fs * fd);
  };
  auto step = [&](int vsi, StepRows& cur, StepRows& nxt) __attribute__((always_inline)) {
    const int v0 = vsi * VS;
    // dU~ of the step and dv first: its stores go out before the next
    // step's loads, so that waiting for those loads does not wait for them
    if (du_wave) {
      f32x4 a[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
      if constexpr (F16W)
        seg_mfma<1>(a, um0, un0, 1, r, kq,
                    seg<C>([&](int m, int kk) { return s.t[kk][m]; },
                           [&](int kk, int n) { return (float)s.h.dh[kk][n] + (float)s.h.dl[kk][n]; }));
      else
        seg_mfma<1>(a, um0, un0, 1, r, kq,
                    seg<C>([&](int m, int kk) { return s.t[kk][m]; }, [&](int kk, int n) { return s.w.du[kk][n]; }));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = um0[0] + 4 * kq + i;
        const int col = un0[0] + r;
        if (row < nval) stx<TIn>(p.dv, dvb + (int64_t)row * p.sdv[1] + v0 + col, s.bt[row] * a[0][i]);
        const float vv = F16W ? (float)s.h.v[row][col] : s.w.v[row][col];
        vu_acc[i] = __builtin_fmaf(vv, a[0][i], vu_acc[i]);
      }
    }
    if (vsi + 2 < nvs) load_step(nxt, vsi + 2);
    // Products contracted over the step's V columns, all of the form
    // X[m][v] Y[n][v]: the contraction runs in 16-column groups in which
    // lane (r, kq) covers columns 4 kq .. 4 kq + 3 over four MFMA steps, so
    // each operand is one 16-byte read per four steps.
    if constexpr (F16W) {
      // lane (r, kq) supplies 8 consecutive columns 8 kq .. of its row; the
      // accumulators keep the layout of the fp32 products below
      const int c8 = 8 * kq;
#pragma unroll
      for (int g = 0; g < NPW; ++g) {
        if (g < ana) {
          // S[an0 + r][8 kq + j] = S^T[8 kq + j][an0 + r]: transposed reads
          const f16x8 sb = tiles16::frag8_t(s.h.ST, 0, an0[g], r, kq), db = tiles16::frag8_t(s.h.dST, 0, an0[g], r, kq);
          const f16x8 xo = tiles16::frag8(&s.h.dO[am0[g] + r][c8]);
          accW[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8(&s.h.dh[am0[g] + r][c8]), sb, accW[g], 0, 0, 0);
          accW[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8(&s.h.dl[am0[g] + r][c8]), sb, accW[g], 0, 0, 0);
          accQ[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xo, sb, accQ[g], 0, 0, 0);
          accK[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8(&s.h.uh[am0[g] + r][c8]), db, accK[g], 0, 0, 0);
          accK[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8(&s.h.ul[am0[g] + r][c8]), db, accK[g], 0, 0, 0);
        }
      }
      // dO u^T (waves 0-3) or du V^T (waves 4-7; diag(beta) applied when stored)
      const f16x8 xh = tiles16::frag8(wave < 4 ? &s.h.dO[cm0[0] + r][c8] : &s.h.dh[cm0[0] + r][c8]);
      const f16x8 xl = tiles16::frag8(&s.h.dl[cm0[0] + r][c8]);
      const f16x8 yh = tiles16::frag8(wave < 4 ? &s.h.uh[cn0[0] + r][c8] : &s.h.v[cn0[0] + r][c8]);
      const f16x8 yl = tiles16::frag8(&s.h.ul[cn0[0] + r][c8]);
      accC[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xh, yh, accC[0], 0, 0, 0);
      accC[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wave < 4 ? xh : xl, wave < 4 ? yl : yh, accC[0], 0, 0, 0);
      dgc_acc += state_dot(s.h.ST, s.h.dST, 1.f, 1.f);
    } else {
#pragma unroll
      for (int c0 = 0; c0 < VS; c0 += 16) {
        const int cc = c0 + 4 * kq;
#pragma unroll
        for (int g = 0; g < NPW; ++g) {
          if (g < ana) {
            f32x4 sb, db;
            if constexpr (ST16) {
              // S[an0 + r][cc + j] = S^T[cc + j][an0 + r]: transposed reads
              const f16x4 hs = tiles16::frag4_t(s.w.st.h.ST, c0, an0[g], r, kq);
              const f16x4 hd = tiles16::frag4_t(s.w.st.h.dST, c0, an0[g], r, kq);
              const float fs = s.scs[c0], fd = s.scd[c0];
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                sb[j] = (float)hs[j] * fs;
                db[j] = (float)hd[j] * fd;
              }
            } else {
              sb = ld4(s.w.st.f.S, an0[g] + r, cc);
              db = ld4(s.w.st.f.dS, an0[g] + r, cc);
            }
            const f32x4 xa = ld4(s.w.du, am0[g] + r, cc), xo = ld4(s.w.dO, am0[g] + r, cc);
            const f32x4 xu = ld4(s.w.u, am0[g] + r, cc);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              accW[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[j], sb[j], accW[g], 0, 0, 0);
              accQ[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(xo[j], sb[j], accQ[g], 0, 0, 0);
              accK[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(xu[j], db[j], accK[g], 0, 0, 0);
            }
          }
        }
        // dO u^T (waves 0-3) or du (diag(beta) V)^T (waves 4-7)
        const f32x4 xc = wave < 4 ? ld4(s.w.dO, cm0[0] + r, cc) : ld4(s.w.du, cm0[0] + r, cc);
        f32x4 yc = wave < 4 ? ld4(s.w.u, cn0[0] + r, cc) : ld4(s.w.v, cn0[0] + r, cc);
        if (wave >= 4) yc *= s.bt[cn0[0] + r];
#pragma unroll
        for (int j = 0; j < 4; ++j) accC[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(xc[j], yc[j], accC[0], 0, 0, 0);
      }
      if constexpr (ST16) {
        const int v = (tid / (K / 8)) % VS;
        dgc_acc += state_dot(s.w.st.h.ST, s.w.st.h.dST, s.scs[v], s.scd[v]);
      } else {
        for (int e = tid; e < K * VS; e += NTG)
          dgc_acc = __builtin_fmaf(s.w.st.f.S[e / VS][e % VS], s.w.st.f.dS[e / VS][e % VS], dgc_acc);
      }
    }
    __syncthreads();
    if (vsi + 1 < nvs) {
      store_step(cur);
      __syncthreads();
    }
  };
  if constexpr (NVS > 0) {
#pragma unroll
    for (int vsi = 0; vsi < NVS; vsi += 2) {
      step(vsi, rb, ra);
      if (vsi + 1 < NVS) step(vsi + 1, ra, rb);
    }
  } else {
    for (int vsi = 0; vsi < nvs; vsi += 2) {
      step(vsi, rb, ra);
      if (vsi + 1 < nvs) step(vsi + 1, ra, rb);
    }
  }

  // ---- accumulators -> LDS, row partials
#pragma unroll
  for (int i = 0; i < NPW; ++i) {
    if (i < ana) {
      float pq[4], pk[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = am0[i] + 4 * kq + e, col = an0[i] + r;
        s.dw[row][col] = -accW[i][e];
        if constexpr (F16W) {
          const float w = pin(-accW[i][e]);
          s.x.dwh[row][col] = (f16)w;
          s.x.dwl[row][col] = (f16)(w - (float)(f16)w);
        }
        pq[e] = sum16(s.q[row][col] * accQ[i][e]);
        pk[e] = sum16(s.k[row][col] * accK[i][e]);
      }
      if (r == 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s.rq[an0[i] / 16][am0[i] + 4 * kq + e] = pq[e];
          s.rk[an0[i] / 16][am0[i] + 4 * kq + e] = pk[e];
        }
      }
    }
  }
  if constexpr (F16W) {
    for (int e = tid; e < C * C; e += NTG) {
      const float x = pin(s.t[e / C][e % C]);
      s.x.th[e / C][e % C] = (f16)x;
      s.x.tl[e / C][e % C] = (f16)(x - (float)(f16)x);
    }
    // q and k rows in fp16: the raw rows loaded at the start (kept in
    // registers through the walk; rows past the chunk end are zero)
    lq.store_raw(tid, s.x.q);
    lk.store_raw(tid, s.x.k);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int row = cm0[0] + 4 * kq + e, col = cn0[0] + r;
    if (wave < 4) {
      const float y = pin(scale * s.m[row][col] * accC[0][e]);
      s.y[row][col] = y;
      if constexpr (!F16W) s.yp[row][col] = scale * accC[0][e] * s.pm[row][col];
      if constexpr (F16W) {
        s.x.yh[row][col] = (f16)y;
        s.x.yl[row][col] = (f16)(y - (float)(f16)y);
      }
    } else {
      s.dt[row][col] = F16W ? s.bt[col] * accC[0][e] : accC[0][e];
    }
  }
  if (du_wave) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x = sum16(vu_acc[e]);
      if (r == 0) s.vu[un0[0] / 16][um0[0] + 4 * kq + e] = x;
    }
  }
  {
    float x = dgc_acc;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
    if (lane == 0) s.red[wave] = x;
  }
  __syncthreads();
  // dT = du (beta V)^T + dW (beta gam K)^T;  dW~ = T^T dW
  f32x4 aw[NPW];  // fp16 inputs: dW~ in the tiles of accW
  if constexpr (F16W) {
    // fp16 MFMA on hi + lo pairs; transposed operands (T^T, dW columns) by
    // ds_read_b64_tr_b16.  dT: waves 0-3, one 16 x 16 tile each.
    if (wave < 4) {
      const int dm = (wave >> 1) * 16, dn = (wave & 1) * 16;
      f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < K; kb += 32) {
        const f16x8 kf = tiles16::frag8(&s.x.k[dn + r][kb + 8 * kq]);
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8(&s.x.dwh[dm + r][kb + 8 * kq]), kf, a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8(&s.x.dwl[dm + r][kb + 8 * kq]), kf, a, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = dm + 4 * kq + e, col = dn + r;
        const float x = pin(s.dt[row][col] + s.bt[col] * s.gam[col] * a[e]);
        s.dt[row][col] = x;
        s.x.dth[row][col] = (f16)x;
        s.x.dtl[row][col] = (f16)(x - (float)(f16)x);
      }
    } else {
      // K K^T and Q K^T (the 16-bit prep does not store them; exact
      // products of the fp16 rows), one 16 x 16 tile of each per wave:
      // K K^T -> kk, dQK o Q K^T = y o Q K^T -> yp
      const int pm0 = ((wave - 4) >> 1) * 16, pn0 = (wave & 1) * 16;
      f32x4 akk = {0.f, 0.f, 0.f, 0.f}, aqk = akk;
#pragma unroll
      for (int kb = 0; kb < K; kb += 32) {
        const f16x8 kf = tiles16::frag8(&s.x.k[pn0 + r][kb + 8 * kq]);
        akk = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8(&s.x.k[pm0 + r][kb + 8 * kq]), kf, akk, 0, 0, 0);
        aqk = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8(&s.x.q[pm0 + r][kb + 8 * kq]), kf, aqk, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = pm0 + 4 * kq + e, col = pn0 + r;
        s.kk[row][col] = akk[e];
        s.yp[row][col] = s.y[row][col] * aqk[e];
      }
    }
#pragma unroll
    for (int g = 0; g < NPW; ++g) {
      aw[g] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (g < ana) {
        const f16x8 th = tiles16::frag8_t(s.x.th, 0, am0[g], r, kq), tl = tiles16::frag8_t(s.x.tl, 0, am0[g], r, kq);
        const f16x8 wh = tiles16::frag8_t(s.x.dwh, 0, an0[g], r, kq);
        aw[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(th, wh, aw[g], 0, 0, 0);
        aw[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(th, tiles16::frag8_t(s.x.dwl, 0, an0[g], r, kq), aw[g], 0,
                                                       0, 0);
        aw[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(tl, wh, aw[g], 0, 0, 0);
        float pw[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) pw[e] = sum16(s.k[am0[g] + 4 * kq + e][an0[g] + r] * aw[g][e]);
        if (r == 0) {
#pragma unroll
          for (int e = 0; e < 4; ++e) s.rw[an0[g] / 16][am0[g] + 4 * kq + e] = pw[e];
        }
      }
    }
  } else {
    mmx<NTG, C, C>(tid, [&](int m, int n, float x) { s.dt[m][n] += x; },
                   seg<K>([&](int m, int kk) { return s.dw[m][kk]; },
                          [&](int kk, int n) { return s.bt[n] * s.gam[n] * s.k[n][kk]; }));
    mmx<NTG, C, K>(tid, [&](int m, int n, float x) { s.dwt[m][n] = x; },
                   seg<C>([&](int m, int kk) { return s.t[kk][m]; }, [&](int kk, int n) { return s.dw[kk][n]; }));
  }
  if (tid < C) {
    float a = 0.f, b = 0.f;
    for (int j = 0; j < NCT; ++j) {
      a += s.rq[j][tid];
      b += s.rk[j][tid];
    }
    s.dgam[tid] = scale * a;  // scale dO_t.(Q S)_t
    s.dD[tid] = b;            // u_t.(K dS')_t
  }
  if (tid == 0) {
    float x = 0.f;
    for (int w = 0; w < NTG / 64; ++w) x += s.red[w];
    s.dgC = x;  // <dS', S>
  }
  __syncthreads();
  // Z = T^T dT;  k_t.dW~_t
  if constexpr (F16W) {
    if (wave < 4) {
      const int zm = (wave >> 1) * 16, zn = (wave & 1) * 16;
      const f16x8 th = tiles16::frag8_t(s.x.th, 0, zm, r, kq), dh = tiles16::frag8_t(s.x.dth, 0, zn, r, kq);
      f32x4 a = {0.f, 0.f, 0.f, 0.f};
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(th, dh, a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(th, tiles16::frag8_t(s.x.dtl, 0, zn, r, kq), a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8_t(s.x.tl, 0, zm, r, kq), dh, a, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = zm + 4 * kq + e, col = zn + r;
        const float z = pin(a[e]);
        s.x.zh[row][col] = (f16)z;
        s.x.zl[row][col] = (f16)(z - (float)(f16)z);
      }
    }
    if (tid < C) {
      float x = 0.f;
      for (int j = 0; j < NCT; ++j) x += s.rw[j][tid];
      s.kw[tid] = x;
    }
  } else {
    mmx<NTG, C, C>(tid, [&](int m, int n, float x) { s.z[m][n] = x; },
                   seg<C>([&](int m, int kk) { return s.t[kk][m]; }, [&](int kk, int n) { return s.dt[kk][n]; }));
    const float kw = row_sum<NTG, C, K>(tid, [&](int rr, int i) { return s.k[rr][i] * s.dwt[rr][i]; });
    if (tid % RL == 0) s.kw[tid / RL] = kw;
  }
  __syncthreads();
  // dA = -tril_-1(Z T^T) -> dt
  if constexpr (F16W) {
    if (wave < 4) {
      const int am = (wave >> 1) * 16, an = (wave & 1) * 16;
      const f16x8 zh = tiles16::frag8(&s.x.zh[am + r][8 * kq]), th = tiles16::frag8(&s.x.th[an + r][8 * kq]);
      f32x4 a = {0.f, 0.f, 0.f, 0.f};
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(zh, th, a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(zh, tiles16::frag8(&s.x.tl[an + r][8 * kq]), a, 0, 0, 0);
      a = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8(&s.x.zl[am + r][8 * kq]), th, a, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = am + 4 * kq + e, col = an + r;
        s.dt[row][col] = col < row ? -a[e] : 0.f;
      }
    }
  } else {
    mmx<NTG, C, C>(tid, [&](int m, int n, float x) { s.dt[m][n] = n < m ? -x : 0.f; },
                   seg<C>([&](int m, int kk) { return s.z[m][kk]; }, [&](int kk, int n) { return s.t[n][kk]; }));
  }
  __syncthreads();
  // dKK = dA o beta_t M -> z;  dbeta and db
  for (int e = tid; e < C * C; e += NTG) {
    const int t = e / C, j = e % C;
    s.z[t][j] = j < t ? s.dt[t][j] * s.bt[t] * s.m[t][j] : 0.f;
  }
  {
    auto amat = [&](int t, int j) { return j < t ? s.bt[t] * s.m[t][j] * s.kk[t][j] : 0.f; };
    const float am = row_sum<NTG, C, C>(tid, [&](int rr, int j) { return s.dt[rr][j] * s.m[rr][j] * s.kk[rr][j]; });
    // db_t through M (dQK o QK) and A (dA o A): row sums minus column sums
    const float mt = row_sum<NTG, C, C>(tid, [&](int rr, int j) {
      return s.yp[rr][j] - s.yp[j][rr] + s.dt[rr][j] * amat(rr, j) - s.dt[j][rr] * amat(j, rr);
    });
    const float dd = row_sum<NTG, C, C>(tid, [&](int rr, int j) { return s.dD[j] * s.D[j]; });
    if (tid % RL == 0) {
      const int rr = tid / RL;
      float vu = 0.f;
#pragma unroll
      for (int j = 0; j < VS / 16; ++j) vu += s.vu[j][rr];
      s.dbt[rr] = vu + s.gam[rr] * s.kw[rr] + am;
      const float dgam = s.dgam[rr] + s.bt[rr] * s.kw[rr];
      // ... and through gam, D and (last row) gam_C and every D_j
      float d = mt + dgam * s.gam[rr] - s.dD[rr] * s.D[rr];
      if (rr == C - 1) d += dd + s.dgC * s.gC;
      s.db[rr] = d;
    }
  }
  __syncthreads();
  if constexpr (F16W) {
    // dKK + dKK^T as fp16 pairs for the dk product (published by the
    // barrier below)
    for (int e = tid; e < C * C; e += NTG) {
      const int t = e / C, j = e % C;
      const float zz = pin(s.z[t][j] + s.z[j][t]);
      s.x.zh[t][j] = (f16)zz;
      s.x.zl[t][j] = (f16)(zz - (float)(f16)zz);
    }
  }
  if (wave == 0) {
    // dg_t = sum_{j >= t} db_j: lane l scans db[C - 1 - l]
    const float x = scan32(lane < C ? s.db[C - 1 - lane] : 0.f);
    const int t = C - 1 - lane;
    if (lane < C && t < nval) store_scalar(p.dg, head_base(rs, hi, p.sdg) + (int64_t)(t0 + t) * p.sdg[1], p.g_dtype, x);
  }
  if (tid < nval)
    store_scalar(p.dbeta, head_base(rs, hi, p.sdb) + (int64_t)(t0 + tid) * p.sdb[1], p.beta_dtype, s.dbt[tid]);
  // dq = dQK K + scale diag(gam) dO S^T;
  // dk = dQK^T Q + diag(D) u dS'^T + diag(beta gam) dW~ + (dKK + dKK^T) K
  {
    f32x4 aq[NPW], ak[NPW];
#pragma unroll
    for (int i = 0; i < NPW; ++i) {
      aq[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      ak[i] = aq[i];
    }
    if constexpr (F16W) {
      __syncthreads();  // the dKK + dKK^T pairs
      // lane (r, kq): rows of dQK / dQK^T / dKK + dKK^T (A) and columns of
      // K / Q (B), contraction indices 8 kq .. 8 kq + 7 of the C = 32
#pragma unroll
      for (int g = 0; g < NPW; ++g) {
        if (g < ana) {
          const f16x8 kt = tiles16::frag8_t(s.x.k, 0, an0[g], r, kq);
          const f16x8 qt = tiles16::frag8_t(s.x.q, 0, an0[g], r, kq);
          const int m = am0[g] + r;
          aq[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8(&s.x.yh[m][8 * kq]), kt, aq[g], 0, 0, 0);
          aq[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8(&s.x.yl[m][8 * kq]), kt, aq[g], 0, 0, 0);
          ak[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8_t(s.x.yh, 0, am0[g], r, kq), qt, ak[g], 0,
                                                         0, 0);
          ak[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8_t(s.x.yl, 0, am0[g], r, kq), qt, ak[g], 0,
                                                         0, 0);
          ak[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8(&s.x.zh[m][8 * kq]), kt, ak[g], 0, 0, 0);
          ak[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(tiles16::frag8(&s.x.zl[m][8 * kq]), kt, ak[g], 0, 0, 0);
        }
      }
    } else {
      seg_mfma<NPW>(aq, am0, an0, ana, r, kq,
                    seg<C>([&](int m, int kk) { return s.y[m][kk]; }, [&](int kk, int n) { return s.k[kk][n]; }));
      seg_mfma<NPW>(ak, am0, an0, ana, r, kq,
                    seg<C>([&](int m, int kk) { return s.y[kk][m]; }, [&](int kk, int n) { return s.q[kk][n]; }));
      seg_mfma<NPW>(ak, am0, an0, ana, r, kq,
                    seg<C>([&](int m, int kk) { return s.z[m][kk] + s.z[kk][m]; },
                           [&](int kk, int n) { return s.k[kk][n]; }));
    }
#pragma unroll
    for (int i = 0; i < NPW; ++i) {
      if (i < ana) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = am0[i] + 4 * kq + e, col = an0[i] + r;
          if (row < nval) {
            const float dq = aq[i][e] + scale * s.gam[row] * accQ[i][e];
            const float dwt = F16W ? aw[i][e] : s.dwt[row][col];
            const float dk = ak[i][e] + s.D[row] * accK[i][e] + s.bt[row] * s.gam[row] * dwt;
            stx<TIn>(p.dq, dqb + (int64_t)row * p.sdq[1] + col, dq);
            stx<TIn>(p.dk, dkb + (int64_t)row * p.sdk[1] + col, dk);
          }
        }
      }
    }
  }
}

// Workspace layout (each part 256-byte aligned).
struct Layout {
  int64_t rec, ckS, ckD, uu, du, r16, scl, total;  // offsets in bytes
  int64_t nslot;
};

inline int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// w16: the 16-bit walks (T and the gates in the record, fp16 S and dS').
inline Layout layout(int B, int T, int H, int K, int V, int n_seq, bool w16) {
  Layout L;
  const int64_t nch = (T + C - 1) / C;
  L.nslot = n_seq > 0 ? nch + n_seq : (int64_t)B * nch;
  const int64_t nr = L.nslot * H;
  int64_t off = 0;
  L.rec = off;
  off = align256(off + nr * (w16 ? RecT::SIZE : rec_size(K)) * 4);
  const int64_t sb = w16 ? 2 : 4;  // bytes per element of S and dS'
  L.ckS = off;
  off = align256(off + nr * K * V * sb);
  L.ckD = off;
  off = align256(off + nr * K * V * sb);
  L.uu = off;
  off = align256(off + nr * C * V * 4);
  L.du = off;
  off = align256(off + nr * C * V * 4);
  L.r16 = off;
  if (w16) off = align256(off + nr * rec16_size(K) * 2);
  L.scl = off;  // two floats per walk unit (B sequences x H x V / BV)
  off = align256(off + 2 * (int64_t)B * H * (V / BV) * 4);
  L.total = off;
  return L;
}

template <typename TIn, int K>
int launch_k(const BArgs& a, int64_t nrec, hipStream_t s) {
  if constexpr (!std::is_same<TIn, float>::value) {
    if (nrec > 0) {
      if (a.w16)
        hipLaunchKernelGGL((prep16_kernel<TIn, K>), dim3((unsigned)((nrec + 4 * NRW - 1) / (4 * NRW))), dim3(256), 0,
                           s, a, nrec);
      else
        hipLaunchKernelGGL((prep_kernel<TIn, K>), dim3((unsigned)nrec), dim3(NTP), 0, s, a);
    }
  } else {
    if (nrec > 0) hipLaunchKernelGGL((prep_kernel<TIn, K>), dim3((unsigned)nrec), dim3(NTP), 0, s, a);
  }
  if constexpr (!std::is_same<TIn, float>::value) {
    if (a.w16) hipLaunchKernelGGL((recur16_kernel<TIn, K>), dim3(2 * a.units), dim3(NTP), 0, s, a);
    else hipLaunchKernelGGL((recur_kernel<TIn, K>), dim3(2 * a.units), dim3(NTP), 0, s, a);
  } else {
    hipLaunchKernelGGL((recur_kernel<TIn, K>), dim3(2 * a.units), dim3(NTP), 0, s, a);
  }
  if (nrec > 0) {
    const dim3 grid((unsigned)nrec);
    const bool st16 = !std::is_same<TIn, float>::value && a.w16;
    if (a.V == 128) {
      if (st16) hipLaunchKernelGGL((grad_kernel<TIn, K, 32, true, 4>), grid, dim3(NTG), 0, s, a);
      else hipLaunchKernelGGL((grad_kernel<TIn, K, 32, false, 4>), grid, dim3(NTG), 0, s, a);
    } else if (a.V % 32 == 0) {
      if (st16) hipLaunchKernelGGL((grad_kernel<TIn, K, 32, true, 0>), grid, dim3(NTG), 0, s, a);
      else hipLaunchKernelGGL((grad_kernel<TIn, K, 32, false, 0>), grid, dim3(NTG), 0, s, a);
    } else {
      if (st16) hipLaunchKernelGGL((grad_kernel<TIn, K, 16, true, 0>), grid, dim3(NTG), 0, s, a);
      else hipLaunchKernelGGL((grad_kernel<TIn, K, 16, false, 0>), grid, dim3(NTG), 0, s, a);
    }
  }
  return (int)hipGetLastError();
}

template <typename TIn>
int launch_t(const BArgs& a, int K, int64_t nrec, hipStream_t s) {
  switch (K) {
    case 32: return launch_k<TIn, 32>(a, nrec, s);
    case 64: return launch_k<TIn, 64>(a, nrec, s);
    case 128: return launch_k<TIn, 128>(a, nrec, s);
    default: return GDN_ERR_UNSUPPORTED;
  }
}

}  // namespace bwd
}  // namespace gdn

using namespace gdn;

// The 16-bit walks: 16-bit q, k, v with dO of the same type, whose rows
// take 4-byte element-pair loads.
static bool bwd_w16(const GdnBwdParams& P) {
  return P.qkv_dtype != GDN_DTYPE_F32 && P.do_dtype == P.qkv_dtype &&
         reinterpret_cast<uintptr_t>(P.d_o) % 4 == 0 && P.do_stride[0] % 2 == 0 && P.do_stride[1] % 2 == 0 &&
         P.do_stride[2] % 2 == 0;
}

namespace gdn {
namespace bwd {

// Segments.  The workspace of one pass holds every chunk's S, dS', u and du
// (about 108 KB per (chunk, head) with the 16-bit walks at K = V = 128), so
// it grows with T.  A dense batch of more than kSegChunks chunks per
// sequence runs in segments of L chunks instead, last segment first:
//   1. a forward pass over segments 0 .. n-2 (gdn_fwd_launch, one call per
//      segment, o into scratch) leaves the fp32 state at the start of every
//      later segment (the checkpoints);
//   2. segment j's backward starts from checkpoint j (h0 for j = 0) and takes
//      as the gradient of its final state the gradient of its successor's
//      initial state (d_final_state for the last segment); its dh0 is
//      carried to segment j - 1 (the caller's dh0 for j = 0).
// The chunk gradients are independent given S and dS' at the segment ends,
// so the segments add up to the one-pass backward.  The workspace is one
// segment's layout (the forward pass's records and o scratch reuse it) plus
// n + 1 states of B H K V floats.  The segment length is what the caller's
// workspace holds, as for the forward.
constexpr int64_t kSegChunks = 256;

struct SegPlan {
  int64_t L = 0, nseg = 0;  // chunks per segment, segments
  int64_t region = 0;       // one segment's layout, or the forward pass's scratch
  int64_t fwd_ws = 0;       // forward workspace, at offset 0 of the region
  int64_t fwd_o = 0;        // forward o scratch offset
  int64_t state_bytes = 0;  // one fp32 [B, H, K, V] state, 256-byte aligned
  int64_t ckpt = 0;         // nseg - 1 checkpoints
  int64_t carry = 0;        // two state gradients (in, out)
  int64_t total = 0;
};

// Forward params over rows [t0, t0 + Tn) of P's inputs, o into `o` (dense,
// the input dtype), the state from h0 (h0_stride) into fs (dense).
inline GdnFwdParams fwd_params(const GdnBwdParams& P, int64_t t0, int Tn, const float* h0, const int64_t* h0s,
                               float* fs, void* o) {
  GdnFwdParams f = {};
  const int eq = elem_bytes(P.qkv_dtype), eg = elem_bytes(P.g_dtype), eb = elem_bytes(P.beta_dtype);
  auto off = [](const void* p, int64_t t0, const int64_t* st, int e) {
    return p ? static_cast<const void*>(static_cast<const char*>(p) + t0 * st[1] * e) : nullptr;
  };
  f.q = off(P.q, t0, P.q_stride, eq);
  f.k = off(P.k, t0, P.k_stride, eq);
  f.v = off(P.v, t0, P.v_stride, eq);
  f.g = off(P.g, t0, P.g_stride, eg);
  f.beta = off(P.beta, t0, P.beta_stride, eb);
  f.h0 = h0;
  f.o = o;
  f.final_state = fs;
  for (int d = 0; d < 3; ++d) {
    f.q_stride[d] = P.q_stride[d];
    f.k_stride[d] = P.k_stride[d];
    f.v_stride[d] = P.v_stride[d];
    f.g_stride[d] = P.g_stride[d];
    f.beta_stride[d] = P.beta_stride[d];
  }
  f.o_stride[0] = (int64_t)Tn * P.H * P.V;
  f.o_stride[1] = (int64_t)P.H * P.V;
  f.o_stride[2] = P.V;
  for (int d = 0; d < 4; ++d) f.h0_stride[d] = h0s ? h0s[d] : 0;
  f.fs_stride[0] = (int64_t)P.H * P.K * P.V;
  f.fs_stride[1] = (int64_t)P.K * P.V;
  f.fs_stride[2] = P.V;
  f.fs_stride[3] = 1;
  f.B = P.B;
  f.T = Tn;
  f.H = P.H;
  f.K = P.K;
  f.V = P.V;
  f.scale = 1.f;
  f.chunk_size = C;
  f.qkv_dtype = P.qkv_dtype;
  f.g_dtype = P.g_dtype;
  f.beta_dtype = P.beta_dtype;
  f.o_dtype = P.qkv_dtype;
  return f;
}

// The workspace of a dense call run in segments of L chunks (L >= the
// call's chunk count: one pass, the plain layout).
inline SegPlan seg_plan(const GdnBwdParams& P, bool w16, int64_t L) {
  SegPlan sp;
  const int64_t nch = (P.T + C - 1) / C;
  sp.L = L < nch ? L : nch;
  if (sp.L < 1) sp.L = 1;
  sp.nseg = nch > 0 ? (nch + sp.L - 1) / sp.L : 1;
  const int Tseg = (int)(sp.nseg > 1 ? sp.L * C : P.T);
  const int64_t lay = layout(P.B, Tseg, P.H, P.K, P.V, 0, w16).total;
  if (sp.nseg == 1) {
    sp.region = sp.total = lay;
    return sp;
  }
  GdnFwdParams f = fwd_params(P, 0, Tseg, nullptr, nullptr, nullptr, nullptr);
  sp.fwd_ws = align256(gdn_fwd_workspace_size(&f));
  sp.fwd_o = sp.fwd_ws;
  const int64_t need = sp.fwd_o + align256((int64_t)P.B * Tseg * P.H * P.V * elem_bytes(P.qkv_dtype));
  sp.region = lay > need ? lay : need;
  sp.state_bytes = align256((int64_t)P.B * P.H * P.K * P.V * 4);
  sp.ckpt = sp.region;
  sp.carry = sp.ckpt + (sp.nseg - 1) * sp.state_bytes;
  sp.total = sp.carry + 2 * sp.state_bytes;
  return sp;
}

}  // namespace bwd
}  // namespace gdn

extern "C" int64_t gdn_bwd_workspace_size(int B, int T, int H, int K, int V, int n_seq) {
  if (B <= 0 || T < 0 || H <= 0 || V <= 0 || V % bwd::BV != 0 || n_seq < 0) return -1;
  if (K != 32 && K != 64 && K != 128) return -1;
  const int64_t nch = ((int64_t)T + bwd::C - 1) / bwd::C;
  if (n_seq > 0 || nch <= bwd::kSegChunks) {
    const int64_t a = bwd::layout(B, T, H, K, V, n_seq, false).total, b = bwd::layout(B, T, H, K, V, n_seq, true).total;
    return a > b ? a : b;  // enough for either path
  }
  // segments of kSegChunks chunks: the largest plan over the dtypes
  int64_t best = 0;
  for (int dt : {GDN_DTYPE_F32, GDN_DTYPE_F16, GDN_DTYPE_BF16}) {
    GdnBwdParams P = {};
    P.B = B; P.T = T; P.H = H; P.K = K; P.V = V;
    P.qkv_dtype = dt; P.g_dtype = GDN_DTYPE_F32; P.beta_dtype = GDN_DTYPE_F32;
    for (bool w16 : {false, true}) {
      if (w16 && dt == GDN_DTYPE_F32) continue;
      const int64_t t = bwd::seg_plan(P, w16, bwd::kSegChunks).total;
      if (t < 0) return -1;
      best = t > best ? t : best;
    }
  }
  return best;
}

// The workspace of a call run in segments of at most `seg_chunks` chunks.
static int64_t bwd_workspace_bytes(const GdnBwdParams* prm, int64_t seg_chunks) {
  if (prm == nullptr) return -1;
  const GdnBwdParams& P = *prm;
  if (P.B <= 0 || P.T < 0 || P.H <= 0 || P.V <= 0 || P.V % bwd::BV != 0) return -1;
  if (P.K != 32 && P.K != 64 && P.K != 128) return -1;
  if (!valid_dtype(P.qkv_dtype) || !valid_dtype(P.do_dtype)) return -1;
  if (P.cu_seqlens) return bwd::layout(P.B, P.T, P.H, P.K, P.V, P.B, bwd_w16(P)).total;
  return bwd::seg_plan(P, bwd_w16(P), seg_chunks).total;
}

extern "C" int64_t gdn_bwd_workspace_size_params(const GdnBwdParams* prm) {
  return bwd_workspace_bytes(prm, bwd::kSegChunks);
}

extern "C" int64_t gdn_bwd_segment_workspace_size(const GdnBwdParams* prm, int seg_chunks) {
  if (seg_chunks < 1) return -1;
  return bwd_workspace_bytes(prm, seg_chunks);
}

// Arguments every path checks: shapes, dtypes, pointers, alignment.
static int bwd_check(const GdnBwdParams& P) {
  if (P.B <= 0 || P.H <= 0 || P.T < 0 || P.V <= 0 || P.V % bwd::BV != 0) return GDN_ERR_BAD_SHAPE;
  if (P.K != 32 && P.K != 64 && P.K != 128) return GDN_ERR_UNSUPPORTED;
  if (!valid_dtype(P.qkv_dtype) || !valid_dtype(P.g_dtype) || !valid_dtype(P.beta_dtype) ||
      !valid_dtype(P.do_dtype))
    return GDN_ERR_BAD_DTYPE;
  if (P.T > 0 && (P.q == nullptr || P.k == nullptr || P.v == nullptr || P.g == nullptr ||
                  P.beta == nullptr || P.d_o == nullptr || P.dq == nullptr || P.dk == nullptr ||
                  P.dv == nullptr || P.dg == nullptr || P.dbeta == nullptr))
    return GDN_ERR_NULL_POINTER;
  // q, k, v rows are read as 16-byte vectors, as in the forward
  if (P.T > 0) {
    const int eb = elem_bytes(P.qkv_dtype);
    const void* ptrs[3] = {P.q, P.k, P.v};
    const int64_t* strides[3] = {P.q_stride, P.k_stride, P.v_stride};
    for (int i = 0; i < 3; ++i) {
      if (reinterpret_cast<uintptr_t>(ptrs[i]) % 16 != 0) return GDN_ERR_MISALIGNED;
      for (int d = 0; d < 3; ++d)
        if ((strides[i][d] * eb) % 16 != 0) return GDN_ERR_MISALIGNED;
    }
  }
  return GDN_OK;
}

// One pass over the whole of P (the kernels' workspace at P.workspace).
static int bwd_launch_one(const GdnBwdParams& P, hipStream_t s) {
  const int64_t units = (int64_t)P.B * P.H * (P.V / bwd::BV);
  // B is the number of sequences when cu_seqlens is given (one packed batch)
  const bool w16 = bwd_w16(P);
  const bwd::Layout L = bwd::layout(P.B, P.T, P.H, P.K, P.V, P.cu_seqlens ? P.B : 0, w16);
  const int64_t nrec = L.nslot * P.H;
  if (2 * units > 0x7fffffffLL || nrec > 0x7fffffffLL || (int64_t)P.B * P.T * P.H * P.K >= (1LL << 40))
    return GDN_ERR_BAD_SHAPE;
  if (P.workspace == nullptr || reinterpret_cast<uintptr_t>(P.workspace) % 256 != 0 ||
      P.workspace_bytes < L.total)
    return GDN_ERR_WORKSPACE;
  if (P.T == 0 && P.dh0 == nullptr) return GDN_OK;

  char* ws = static_cast<char*>(P.workspace);
  bwd::BArgs a = {};
  a.q = P.q; a.k = P.k; a.v = P.v; a.g = P.g; a.beta = P.beta; a.h0 = P.h0;
  a.d_o = P.d_o; a.dfs = P.d_final_state;
  a.dq = P.dq; a.dk = P.dk; a.dv = P.dv; a.dg = P.dg; a.dbeta = P.dbeta; a.dh0 = P.dh0;
  a.rec = reinterpret_cast<float*>(ws + L.rec);
  a.ckS = reinterpret_cast<float*>(ws + L.ckS);
  a.ckD = reinterpret_cast<float*>(ws + L.ckD);
  a.uu = reinterpret_cast<float*>(ws + L.uu);
  a.du = reinterpret_cast<float*>(ws + L.du);
  a.r16 = reinterpret_cast<f16*>(ws + L.r16);
  a.scl = reinterpret_cast<float*>(ws + L.scl);
  for (int d = 0; d < 3; ++d) {
    a.sq[d] = P.q_stride[d]; a.sk[d] = P.k_stride[d]; a.sv[d] = P.v_stride[d];
    a.sg[d] = P.g_stride[d]; a.sb[d] = P.beta_stride[d]; a.sdo[d] = P.do_stride[d];
    a.sdq[d] = P.dq_stride[d]; a.sdk[d] = P.dk_stride[d]; a.sdv[d] = P.dv_stride[d];
    a.sdg[d] = P.dg_stride[d]; a.sdb[d] = P.dbeta_stride[d];
  }
  for (int d = 0; d < 4; ++d) {
    a.sh0[d] = P.h0_stride[d]; a.sdfs[d] = P.dfs_stride[d]; a.sdh0[d] = P.dh0_stride[d];
  }
  a.B = P.B; a.T = P.T; a.H = P.H; a.V = P.V; a.nv = P.V / bwd::BV;
  a.nchmax = (P.T + bwd::C - 1) / bwd::C;
  a.units = (int)units;
  a.scale = P.scale;
  a.g_dtype = P.g_dtype; a.beta_dtype = P.beta_dtype; a.do_dtype = P.do_dtype;
  a.cu = P.cu_seqlens;
  a.xcd_remap = (units % 8 == 0) ? 1 : 0;
  // fp16 pair recurrences (the 16-bit walks)
  a.w16 = w16;

  const int64_t nrec_launch = P.T > 0 ? nrec : 0;
  switch (P.qkv_dtype) {
    case GDN_DTYPE_F16: return bwd::launch_t<f16>(a, P.K, nrec_launch, s);
    case GDN_DTYPE_BF16: return bwd::launch_t<bf16_t>(a, P.K, nrec_launch, s);
    default: return bwd::launch_t<float>(a, P.K, nrec_launch, s);
  }
}

extern "C" int gdn_bwd_launch(const GdnBwdParams* prm, void* stream) {
  if (prm == nullptr) return GDN_ERR_NULL_POINTER;
  const GdnBwdParams& P = *prm;
  const int chk = bwd_check(P);
  if (chk != GDN_OK) return chk;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t nch = ((int64_t)P.T + bwd::C - 1) / bwd::C;
  const bool w16 = bwd_w16(P);
  // one pass: packed sequences, or a workspace that holds every chunk
  if (P.cu_seqlens != nullptr || nch <= 1 || P.workspace == nullptr ||
      P.workspace_bytes >= bwd::layout(P.B, P.T, P.H, P.K, P.V, 0, w16).total)
    return bwd_launch_one(P, s);
  if (reinterpret_cast<uintptr_t>(P.workspace) % 256 != 0) return GDN_ERR_WORKSPACE;
  // the longest segments whose layout fits, then shorter ones until the
  // checkpoints fit beside it
  int64_t lo = 0, hi = nch - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) / 2;
    if (bwd::seg_plan(P, w16, mid).region <= P.workspace_bytes)
      lo = mid;
    else
      hi = mid - 1;
  }
  int64_t L = lo;
  while (L >= 1 && bwd::seg_plan(P, w16, L).total > P.workspace_bytes) --L;
  if (L < 1) return GDN_ERR_WORKSPACE;
  const bwd::SegPlan sp = bwd::seg_plan(P, w16, L);
  char* ws = static_cast<char*>(P.workspace);
  const int64_t dense[4] = {(int64_t)P.H * P.K * P.V, (int64_t)P.K * P.V, P.V, 1};
  auto ckpt = [&](int64_t j) { return reinterpret_cast<float*>(ws + sp.ckpt + j * sp.state_bytes); };
  auto carry = [&](int64_t j) { return reinterpret_cast<float*>(ws + sp.carry + (j & 1) * sp.state_bytes); };
  const int64_t R = sp.L * bwd::C;  // rows per segment
  // 1. the state at the start of segments 1 .. n-1
  for (int64_t j = 0; j + 1 < sp.nseg; ++j) {
    GdnFwdParams f = bwd::fwd_params(P, j * R, (int)R, j == 0 ? P.h0 : ckpt(j - 1), j == 0 ? P.h0_stride : dense,
                                     ckpt(j), ws + sp.fwd_o);
    f.workspace = sp.fwd_ws > 0 ? ws : nullptr;
    f.workspace_bytes = sp.fwd_ws;
    const int st = gdn_fwd_launch(&f, stream);
    if (st != GDN_OK) return st;
  }
  // 2. the segments' backward, last first, the state gradient carried
  const int eq = elem_bytes(P.qkv_dtype), eg = elem_bytes(P.g_dtype), eb = elem_bytes(P.beta_dtype),
            ed = elem_bytes(P.do_dtype);
  for (int64_t j = sp.nseg - 1; j >= 0; --j) {
    const int64_t t0 = j * R;
    GdnBwdParams Q = P;
    auto in = [t0](const void* p, const int64_t* st, int e) {
      return static_cast<const void*>(static_cast<const char*>(p) + t0 * st[1] * e);
    };
    auto out = [t0](void* p, const int64_t* st, int e) {
      return static_cast<void*>(static_cast<char*>(p) + t0 * st[1] * e);
    };
    Q.q = in(P.q, P.q_stride, eq);
    Q.k = in(P.k, P.k_stride, eq);
    Q.v = in(P.v, P.v_stride, eq);
    Q.g = in(P.g, P.g_stride, eg);
    Q.beta = in(P.beta, P.beta_stride, eb);
    Q.d_o = in(P.d_o, P.do_stride, ed);
    Q.dq = out(P.dq, P.dq_stride, eq);
    Q.dk = out(P.dk, P.dk_stride, eq);
    Q.dv = out(P.dv, P.dv_stride, eq);
    Q.dg = out(P.dg, P.dg_stride, eg);
    Q.dbeta = out(P.dbeta, P.dbeta_stride, eb);
    Q.T = (int)(P.T - t0 < R ? P.T - t0 : R);
    if (j > 0) {
      Q.h0 = ckpt(j - 1);
      for (int d = 0; d < 4; ++d) Q.h0_stride[d] = dense[d];
      Q.dh0 = carry(j);
      for (int d = 0; d < 4; ++d) Q.dh0_stride[d] = dense[d];
    }
    if (j + 1 < sp.nseg) {
      Q.d_final_state = carry(j + 1);
      for (int d = 0; d < 4; ++d) Q.dfs_stride[d] = dense[d];
    }
    Q.workspace = ws;
    Q.workspace_bytes = sp.region;
    const int st = bwd_launch_one(Q, s);
    if (st != GDN_OK) return st;
  }
  return GDN_OK;
}
