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
// gdn_ref.py:3-9).
//
// One workgroup per (b, h, 16-column V-slice), 512 threads, everything in
// fp32 in LDS.  Pass 1 walks the chunks forward from h0 and stores the state
// at each chunk start in the workspace; pass 2 walks them backward carrying
// dS.  The K-side terms (dq, dk, dbeta, dg) are sums over V, so each slice
// writes its partial sums to the workspace and a second kernel adds the
// slices (fixed order: deterministic).  Products run on fp32 MFMA with
// operands read from LDS through accessors (the forward's fp16 pipeline is
// not reused here).

#include "gdn_fwd_kernel.h"

namespace gdn {
namespace bwd {

constexpr int C = 32;
constexpr int BV = 16;
constexpr int NT = 512;  // 8 waves: 2 per SIMD (256 VGPRs each)
constexpr int RL = NT / C;  // lanes per row in row reductions
static_assert(RL >= 1 && RL <= 64 && (RL & (RL - 1)) == 0, "row lanes");

struct BArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  const float* h0;
  const void* d_o;
  const float* dfs;
  void* dv;
  float* dh0;
  float* ckpt;
  float* pq;
  float* pk;
  float* pg;
  float* pb;
  int64_t sq[3], sk[3], sv[3], sg[3], sb[3], sdo[3], sdv[3];
  int64_t sh0[4], sdfs[4], sdh0[4];
  int64_t R;  // rows of the partial buffers: B T, or T for packed sequences
  int B, T, H, V, nv;
  float scale;
  int g_dtype, beta_dtype, do_dtype;
  const int64_t* cu;
  int xcd_remap;
};

struct RArgs {
  const float* pq;
  const float* pk;
  const float* pg;
  const float* pb;
  void* dq;
  void* dk;
  void* dg;
  void* dbeta;
  int64_t sdq[3], sdk[3], sdg[3], sdb[3];
  int64_t R;
  int T, H, K, nv;
  int qkv_dtype, g_dtype, beta_dtype;
};

template <int K>
struct alignas(16) BSmem {
  static constexpr int KD = K + 1, BD = BV + 1, CD = C + 1;
  float q[C][KD], k[C][KD], w[C][KD], dw[C][KD];
  float x[C][KD];  // dW~, then the new dS as [K][BD]
  float v[C][BD], dO[C][BD], u[C][BD], du[C][BD], u2[C][BD], qs[C][BD];
  float S[K][BD], dS[K][BD];
  float kk[C][CD], qk[C][CD], m[C][CD], a[C][CD], t[C][CD], dt[C][CD], y[C][CD], z[C][CD];
  float gl[C], bt[C], b[C], gam[C], D[C], dgam[C], dD[C], dbt[C], db[C];
  float red[NT / 64];
  float gC, dgC;
};
static_assert(C * (128 + 1) >= 128 * (BV + 1), "x holds a K x BD tile");

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

// out(m, n, sum over the segments) for an M x N result on the matrix cores
// (v_mfma_f32_16x16x4_f32, full fp32): 16 x 16 output tiles dealt round-robin
// to the waves, up to G of them in
// flight per wave so that their operand loads and MFMA chains overlap.
// Lane l supplies a(m0 + l % 16, k0 + l / 16) and b(k0 + l / 16, n0 + l % 16)
// and receives rows m0 + 4 (l / 16) + i, column n0 + l % 16 of a tile.
template <int G, int KD, typename FA, typename FB>
__device__ __forceinline__ void seg_mfma(f32x4 (&acc)[G], const int (&m0)[G], const int (&n0)[G],
                                         int ng, int r, int kq, const Seg<KD, FA, FB>& s) {
  static_assert(KD % 4 == 0, "contraction length");
#pragma unroll 2
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

template <int M, int N, typename FO, typename... Segs>
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
    (seg_mfma<G>(acc, m0, n0, ng, r, kq, segs), ...);
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (g < ng) {
#pragma unroll
        for (int i = 0; i < 4; ++i) out(m0[g] + 4 * kq + i, n0[g] + r, acc[g][i]);
      }
  }
}

// sum_{i < LEN} f(r, i) for row r = tid / RL, computed by the RL lanes of
// the row (a power of two inside one wave) and returned to all of them.
template <int LEN, typename F>
__device__ __forceinline__ float row_sum(int tid, F&& f) {
  const int r = tid / RL, part = tid % RL;
  float acc = 0.f;
  for (int i = part; i < LEN; i += RL) acc += f(r, i);
#pragma unroll
  for (int o = RL / 2; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
  return acc;
}

template <typename TIn, int K>
__global__ __launch_bounds__(NT) void bwd_kernel(const BArgs p) {
  using Sm = BSmem<K>;
  constexpr int BD = Sm::BD;
  static_assert(K == 32 || K == 64 || K == 128, "K");

  __shared__ Sm s;
  // The thread index is re-read as an opaque value at the top of every
  // chunk iteration, so that per-thread LDS addresses are recomputed there
  // instead of being hoisted out of the chunk loops and held in registers.
  const int tid0 = threadIdx.x;
  const int lane = tid0 & 63, wave = tid0 >> 6;

  int unit = blockIdx.x;
  if (p.xcd_remap) unit = (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3);
  const int vs = unit % p.nv;
  const int bh = unit / p.nv;
  const int bi = bh / p.H;
  const int hi = bh % p.H;
  const int v0 = vs * BV;
  const RowSpan rs = row_span(p.cu, p.T, bi);
  const int Tn = rs.T;
  const int nch = (Tn + C - 1) / C;
  const float scale = p.scale;

  const int64_t qb = head_base(rs, hi, p.sq), kb = head_base(rs, hi, p.sk);
  const int64_t vb = head_base(rs, hi, p.sv) + v0, dob = head_base(rs, hi, p.sdo) + v0;
  const int64_t gb = head_base(rs, hi, p.sg), bb = head_base(rs, hi, p.sb);
  const int64_t dvb = head_base(rs, hi, p.sdv) + v0;
  // rows of the partial buffers ([nv][R][H](K)): b T + t; row t of this
  // chunk sequence starts at pq_h + t H K (pg_h + t H for the gates)
  const int64_t prow0 = rs.b * p.T + rs.t0;
  const int64_t hk = (int64_t)p.H * K;
  float* const pq_h = p.pq + ((int64_t)vs * p.R + prow0) * hk + (int64_t)hi * K;
  float* const pk_h = p.pk + ((int64_t)vs * p.R + prow0) * hk + (int64_t)hi * K;
  float* const pg_h = p.pg + ((int64_t)vs * p.R + prow0) * p.H + hi;
  float* const pb_h = p.pb + ((int64_t)vs * p.R + prow0) * p.H + hi;
  // chunk-start states: slot (chunk) x H x nv x [K][BV]; packed sequence i
  // starts at slot floor(t0 / C) + i, which keeps sequences disjoint.
  const int64_t slot0 = p.cu ? rs.t0 / C + bi : (int64_t)bi * ((p.T + C - 1) / C);
  const int64_t ck_stride = (int64_t)p.H * p.nv * K * BV;
  float* const ck0 = p.ckpt + ((slot0 * p.H + hi) * p.nv + vs) * (int64_t)(K * BV);

  // Chunk rows -> LDS as fp32.  q, k, v move as 16-byte vectors (their rows
  // are 16-byte aligned: the host checks it); every global load of the
  // chunk is issued before the first LDS store.
  constexpr int VEC = 16 / (int)sizeof(TIn);
  constexpr int RVK = K / VEC, NVK = (C * RVK + NT - 1) / NT;
  constexpr int RVV = BV / VEC;
  constexpr int NDO = (C * BV + NT - 1) / NT;
  static_assert(C * RVV <= NT, "v vectors");
  const TIn* const qg = static_cast<const TIn*>(p.q) + qb;
  const TIn* const kg = static_cast<const TIn*>(p.k) + kb;
  const TIn* const vg = static_cast<const TIn*>(p.v) + vb;
  auto load_chunk = [&](int tid, int c, bool full) __attribute__((always_inline)) {
    const int t0 = c * C;
    const u32x4 z = {0u, 0u, 0u, 0u};
    u32x4 rk[NVK], rq[NVK], rv = z;
    float rdo[NDO], rg = 0.f, rb = 0.f;
#pragma unroll
    for (int i = 0; i < NVK; ++i) {
      const int e = tid + i * NT, t = e / RVK, col = (e % RVK) * VEC;
      const bool ok = e < C * RVK && t0 + t < Tn;
      rk[i] = ok ? *reinterpret_cast<const u32x4*>(kg + (int64_t)(t0 + t) * p.sk[1] + col) : z;
      rq[i] = (ok && full) ? *reinterpret_cast<const u32x4*>(qg + (int64_t)(t0 + t) * p.sq[1] + col) : z;
    }
    if (tid < C * RVV) {
      const int t = tid / RVV, col = (tid % RVV) * VEC;
      if (t0 + t < Tn) rv = *reinterpret_cast<const u32x4*>(vg + (int64_t)(t0 + t) * p.sv[1] + col);
    }
#pragma unroll
    for (int i = 0; i < NDO; ++i) {
      const int e = tid + i * NT, t = e / BV, c2 = e % BV;
      rdo[i] = (full && e < C * BV && t0 + t < Tn)
                   ? load_scalar(p.d_o, dob + (int64_t)(t0 + t) * p.sdo[1] + c2, p.do_dtype)
                   : 0.f;
    }
    if (tid < C && t0 + tid < Tn) {
      rg = load_scalar(p.g, gb + (int64_t)(t0 + tid) * p.sg[1], p.g_dtype);
      rb = load_scalar(p.beta, bb + (int64_t)(t0 + tid) * p.sb[1], p.beta_dtype);
    }
#pragma unroll
    for (int i = 0; i < NVK; ++i) {
      const int e = tid + i * NT, t = e / RVK, col = (e % RVK) * VEC;
      if (e < C * RVK) {
        float x[VEC];
        unpack16<TIn>(rk[i], x);
#pragma unroll
        for (int j = 0; j < VEC; ++j) s.k[t][col + j] = x[j];
        if (full) {
          unpack16<TIn>(rq[i], x);
#pragma unroll
          for (int j = 0; j < VEC; ++j) s.q[t][col + j] = x[j];
        }
      }
    }
    if (tid < C * RVV) {
      const int t = tid / RVV, col = (tid % RVV) * VEC;
      float x[VEC];
      unpack16<TIn>(rv, x);
#pragma unroll
      for (int j = 0; j < VEC; ++j) s.v[t][col + j] = x[j];
    }
    if (full) {
#pragma unroll
      for (int i = 0; i < NDO; ++i) {
        const int e = tid + i * NT;
        if (e < C * BV) s.dO[e / BV][e % BV] = rdo[i];
      }
    }
    if (tid < C) {
      s.gl[tid] = rg;
      s.bt[tid] = rb;
    }
  };

  // Gates, M, K K^T (and Q K^T), A, T = (I + A)^-1, W, U, u.  Leaves
  // U in u2.  Starts and ends on a barrier.
  auto chunk_forward = [&](int tid, bool full) __attribute__((always_inline)) {
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
    mmx<C, C>(tid, [&](int m, int n, float x) { s.kk[m][n] = x; },
                   seg<K>([&](int m, int kk) { return s.k[m][kk]; }, [&](int kk, int n) { return s.k[n][kk]; }));
    if (full)
      mmx<C, C>(tid, [&](int m, int n, float x) { s.qk[m][n] = x; },
                     seg<K>([&](int m, int kk) { return s.q[m][kk]; }, [&](int kk, int n) { return s.k[n][kk]; }));
    __syncthreads();
    for (int e = tid; e < C * C; e += NT) {
      const int t = e / C, j = e % C;
      const float mv = j <= t ? expf(s.b[t] - s.b[j]) : 0.f;
      s.m[t][j] = mv;
      s.a[t][j] = j < t ? s.bt[t] * mv * s.kk[t][j] : 0.f;
    }
    __syncthreads();
    if (tid < C) {
      // column tid of T by forward substitution, the column in registers
      const int c = tid;
      float col[C];
#pragma unroll
      for (int i = 0; i < C; ++i) {
        float x = (i == c) ? 1.f : 0.f;
#pragma unroll
        for (int j = 0; j < i; ++j) x = __builtin_fmaf(-s.a[i][j], col[j], x);
        col[i] = x;
      }
#pragma unroll
      for (int i = 0; i < C; ++i) s.t[i][c] = col[i];
    }
    __syncthreads();
    mmx<C, K>(tid, [&](int m, int n, float x) { s.w[m][n] = x; },
                       seg<C>([&](int m, int kk) { return s.t[m][kk]; },
                              [&](int kk, int n) { return s.bt[kk] * s.gam[kk] * s.k[kk][n]; }));
    mmx<C, BV>(tid, [&](int m, int n, float x) { s.u2[m][n] = x; },
                    seg<C>([&](int m, int kk) { return s.t[m][kk]; },
                           [&](int kk, int n) { return s.bt[kk] * s.v[kk][n]; }));
    __syncthreads();
    mmx<C, BV>(tid, [&](int m, int n, float x) { s.u[m][n] = s.u2[m][n] - x; },
                    seg<K>([&](int m, int kk) { return s.w[m][kk]; }, [&](int kk, int n) { return s.S[kk][n]; }));
    __syncthreads();
  };

  // ---------------- pass 1: chunk-start states ----------------
  for (int e = tid0; e < K * BV; e += NT) {
    const int kk = e / BV, c2 = e % BV;
    s.S[kk][c2] = p.h0 ? p.h0[bi * p.sh0[0] + hi * p.sh0[1] + kk * p.sh0[2] + (v0 + c2) * p.sh0[3]] : 0.f;
  }
  __syncthreads();
  for (int c = 0; c < nch; ++c) {
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    float* ck = ck0 + c * ck_stride;
    for (int e = 4 * tid; e < K * BV; e += 4 * NT) {
      const int kk = e / BV, c2 = e % BV;
      *reinterpret_cast<f32x4*>(ck + e) = f32x4{s.S[kk][c2], s.S[kk][c2 + 1], s.S[kk][c2 + 2], s.S[kk][c2 + 3]};
    }
    load_chunk(tid, c, false);
    __syncthreads();
    chunk_forward(tid, false);
    mmx<K, BV>(tid, [&](int m, int n, float x) { s.S[m][n] = s.gC * s.S[m][n] + x; },
                        seg<C>([&](int m, int kk) { return s.k[kk][m] * s.D[kk]; },
                               [&](int kk, int n) { return s.u[kk][n]; }));
    __syncthreads();
  }

  // ---------------- pass 2: gradients, last chunk first ----------------
  for (int e = tid0; e < K * BV; e += NT) {
    const int kk = e / BV, c2 = e % BV;
    s.dS[kk][c2] =
        p.dfs ? p.dfs[bi * p.sdfs[0] + hi * p.sdfs[1] + kk * p.sdfs[2] + (v0 + c2) * p.sdfs[3]] : 0.f;
  }
  float* const xs = &s.x[0][0];
  for (int c = nch - 1; c >= 0; --c) {
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    const int t0 = c * C;
    const float* ck = ck0 + c * ck_stride;
    {
      constexpr int NCK = (K * BV / 4 + NT - 1) / NT;
      f32x4 r4[NCK];
#pragma unroll
      for (int i = 0; i < NCK; ++i)
        if (4 * (tid + i * NT) < K * BV) r4[i] = *reinterpret_cast<const f32x4*>(ck + 4 * (tid + i * NT));
#pragma unroll
      for (int i = 0; i < NCK; ++i) {
        const int e = 4 * (tid + i * NT), kk = e / BV, c2 = e % BV;
        if (e < K * BV) {
#pragma unroll
          for (int j = 0; j < 4; ++j) s.S[kk][c2 + j] = r4[i][j];
        }
      }
    }
    load_chunk(tid, c, true);
    __syncthreads();
    chunk_forward(tid, true);

    // K dS' -> u2 (U is no longer needed), Q S -> qs
    mmx<C, BV>(tid, [&](int m, int n, float x) { s.u2[m][n] = x; },
                    seg<K>([&](int m, int kk) { return s.k[m][kk]; }, [&](int kk, int n) { return s.dS[kk][n]; }));
    mmx<C, BV>(tid, [&](int m, int n, float x) { s.qs[m][n] = x; },
                    seg<K>([&](int m, int kk) { return s.q[m][kk]; }, [&](int kk, int n) { return s.S[kk][n]; }));
    __syncthreads();
    // du = scale P^T dO + D o K dS';  dQK = M o (scale dO u^T)
    mmx<C, BV>(tid, [&](int m, int n, float x) { s.du[m][n] = scale * x + s.D[m] * s.u2[m][n]; },
                    seg<C>([&](int m, int kk) { return s.m[kk][m] * s.qk[kk][m]; },
                           [&](int kk, int n) { return s.dO[kk][n]; }));
    mmx<C, C>(tid, [&](int m, int n, float x) { s.y[m][n] = scale * s.m[m][n] * x; },
                   seg<BV>([&](int m, int kk) { return s.dO[m][kk]; }, [&](int kk, int n) { return s.u[n][kk]; }));
    {
      const float dd = row_sum<BV>(tid, [&](int r, int i) { return s.u[r][i] * s.u2[r][i]; });
      const float dg = row_sum<BV>(tid, [&](int r, int i) { return s.dO[r][i] * s.qs[r][i]; });
      if (tid % RL == 0) {
        s.dD[tid / RL] = dd;
        s.dgam[tid / RL] = scale * dg;
      }
    }
    {
      // dgam_C = <dS', S>
      float part = 0.f;
      for (int e = tid; e < K * BV; e += NT) part = __builtin_fmaf(s.dS[e / BV][e % BV], s.S[e / BV][e % BV], part);
      for (int o = 32; o >= 1; o >>= 1) part += __shfl_xor(part, o, 64);
      if (lane == 0) s.red[wave] = part;
    }
    __syncthreads();
    if (tid == 0) {
      float r = 0.f;
      for (int w = 0; w < NT / 64; ++w) r += s.red[w];
      s.dgC = r;
    }
    // dW = -du S^T
    mmx<C, K>(tid, [&](int m, int n, float x) { s.dw[m][n] = -x; },
                       seg<BV>([&](int m, int kk) { return s.du[m][kk]; }, [&](int kk, int n) { return s.S[n][kk]; }));
    __syncthreads();
    // dT = du (beta V)^T + dW (beta gam K)^T;  dW~ = T^T dW -> x;  dU~ = T^T du -> u2
    mmx<C, C>(tid, [&](int m, int n, float x) { s.dt[m][n] = x; },
                   seg<BV>([&](int m, int kk) { return s.du[m][kk]; },
                           [&](int kk, int n) { return s.bt[n] * s.v[n][kk]; }),
                   seg<K>([&](int m, int kk) { return s.dw[m][kk]; },
                          [&](int kk, int n) { return s.bt[n] * s.gam[n] * s.k[n][kk]; }));
    mmx<C, K>(tid, [&](int m, int n, float x) { s.x[m][n] = x; },
                       seg<C>([&](int m, int kk) { return s.t[kk][m]; }, [&](int kk, int n) { return s.dw[kk][n]; }));
    mmx<C, BV>(tid, [&](int m, int n, float x) { s.u2[m][n] = x; },
                    seg<C>([&](int m, int kk) { return s.t[kk][m]; }, [&](int kk, int n) { return s.du[kk][n]; }));
    __syncthreads();
    // Z = T^T dT;  dv = beta dU~;  dbeta, dgam through W~ and U~
    mmx<C, C>(tid, [&](int m, int n, float x) { s.z[m][n] = x; },
                   seg<C>([&](int m, int kk) { return s.t[kk][m]; }, [&](int kk, int n) { return s.dt[kk][n]; }));
    for (int e = tid; e < C * BV; e += NT) {
      const int t = e / BV, c2 = e % BV;
      if (t0 + t < Tn) stx<TIn>(p.dv, dvb + (int64_t)(t0 + t) * p.sdv[1] + c2, s.bt[t] * s.u2[t][c2]);
    }
    {
      const float kw = row_sum<K>(tid, [&](int r, int i) { return s.k[r][i] * s.x[r][i]; });
      const float vu = row_sum<BV>(tid, [&](int r, int i) { return s.v[r][i] * s.u2[r][i]; });
      if (tid % RL == 0) {
        const int r = tid / RL;
        s.dbt[r] = vu + s.gam[r] * kw;
        s.dgam[r] += s.bt[r] * kw;
      }
    }
    __syncthreads();
    // dA = -tril_-1(Z T^T) -> dt
    mmx<C, C>(tid, [&](int m, int n, float x) { s.dt[m][n] = n < m ? -x : 0.f; },
                   seg<C>([&](int m, int kk) { return s.z[m][kk]; }, [&](int kk, int n) { return s.t[n][kk]; }));
    __syncthreads();
    // dKK = dA o beta_t M -> z;  dbeta += sum_j dA M KK
    for (int e = tid; e < C * C; e += NT) {
      const int t = e / C, j = e % C;
      s.z[t][j] = j < t ? s.dt[t][j] * s.bt[t] * s.m[t][j] : 0.f;
    }
    {
      const float am = row_sum<C>(tid, [&](int r, int j) { return s.dt[r][j] * s.m[r][j] * s.kk[r][j]; });
      // db_t through M (dQK o QK) and A (dA o A): row sums minus column sums
      const float mt = row_sum<C>(tid, [&](int r, int j) {
        return s.y[r][j] * s.qk[r][j] - s.y[j][r] * s.qk[j][r] + s.dt[r][j] * s.a[r][j] -
               s.dt[j][r] * s.a[j][r];
      });
      const float dd = row_sum<C>(tid, [&](int r, int j) { return s.dD[j] * s.D[j]; });
      if (tid % RL == 0) {
        const int r = tid / RL;
        s.dbt[r] += am;
        // ... and through gam, D and (last row) gam_C and every D_j
        float d = mt + s.dgam[r] * s.gam[r] - s.dD[r] * s.D[r];
        if (r == C - 1) d += dd + s.dgC * s.gC;
        s.db[r] = d;
      }
    }
    __syncthreads();
    if (tid < C && t0 + tid < Tn) {
      float acc = 0.f;
      for (int j = tid; j < C; ++j) acc += s.db[j];
      const int64_t r = (int64_t)(t0 + tid) * p.H;
      pg_h[r] = acc;
      pb_h[r] = s.dbt[tid];
    }
    // dq (partial) = dQK K + scale gam dO S^T
    mmx<C, K>(
        tid, [&](int m, int n, float x) {
          if (t0 + m < Tn) pq_h[(int64_t)(t0 + m) * hk + n] = x;
        },
        seg<C>([&](int m, int kk) { return s.y[m][kk]; }, [&](int kk, int n) { return s.k[kk][n]; }),
        seg<BV>([&](int m, int kk) { return scale * s.gam[m] * s.dO[m][kk]; },
                [&](int kk, int n) { return s.S[n][kk]; }));
    // dk (partial) = dQK^T Q + D u dS'^T + (dKK + dKK^T) K + beta gam dW~
    mmx<C, K>(
        tid, [&](int m, int n, float x) {
          if (t0 + m < Tn)
            pk_h[(int64_t)(t0 + m) * hk + n] =
                x + s.bt[m] * s.gam[m] * s.x[m][n];
        },
        seg<C>([&](int m, int kk) { return s.y[kk][m]; }, [&](int kk, int n) { return s.q[kk][n]; }),
        seg<BV>([&](int m, int kk) { return s.D[m] * s.u[m][kk]; }, [&](int kk, int n) { return s.dS[n][kk]; }),
        seg<C>([&](int m, int kk) { return s.z[m][kk] + s.z[kk][m]; }, [&](int kk, int n) { return s.k[kk][n]; }));
    __syncthreads();
    // dS = scale Q^T diag(gam) dO + gam_C dS' - W^T du -> x as [K][BD]
    mmx<K, BV>(tid, [&](int m, int n, float x) { xs[m * BD + n] = x + s.gC * s.dS[m][n]; },
                        seg<C>([&](int m, int kk) { return scale * s.gam[kk] * s.q[kk][m]; },
                               [&](int kk, int n) { return s.dO[kk][n]; }),
                        seg<C>([&](int m, int kk) { return -s.w[kk][m]; }, [&](int kk, int n) { return s.du[kk][n]; }));
    __syncthreads();
    for (int e = tid; e < K * BV; e += NT) s.dS[e / BV][e % BV] = xs[(e / BV) * BD + e % BV];
  }
  __syncthreads();
  if (p.dh0 != nullptr) {
    for (int e = tid0; e < K * BV; e += NT) {
      const int kk = e / BV, c2 = e % BV;
      p.dh0[bi * p.sdh0[0] + hi * p.sdh0[1] + kk * p.sdh0[2] + (v0 + c2) * p.sdh0[3]] = s.dS[kk][c2];
    }
  }
}

// dq, dk, dg, dbeta = the sums of the slices' partials, in row order.
template <typename TIn>
__global__ __launch_bounds__(256) void reduce_kernel(const RArgs p) {
  const int64_t nrow = p.R * p.H;
  const int64_t n_qk = nrow * p.K;
  const int64_t slab_qk = n_qk, slab_g = nrow;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n_qk + nrow; e += stride) {
    if (e < n_qk) {
      const int64_t kk = e % p.K, rh = e / p.K;
      const int64_t h = rh % p.H, r = rh / p.H;
      const int64_t b = r / p.T, t = r % p.T;
      float sq = 0.f, sk = 0.f;
      for (int vs = 0; vs < p.nv; ++vs) {
        sq += p.pq[vs * slab_qk + e];
        sk += p.pk[vs * slab_qk + e];
      }
      stx<TIn>(p.dq, b * p.sdq[0] + t * p.sdq[1] + h * p.sdq[2] + kk, sq);
      stx<TIn>(p.dk, b * p.sdk[0] + t * p.sdk[1] + h * p.sdk[2] + kk, sk);
    } else {
      const int64_t rh = e - n_qk;
      const int64_t h = rh % p.H, r = rh / p.H;
      const int64_t b = r / p.T, t = r % p.T;
      float sg = 0.f, sb = 0.f;
      for (int vs = 0; vs < p.nv; ++vs) {
        sg += p.pg[vs * slab_g + rh];
        sb += p.pb[vs * slab_g + rh];
      }
      store_scalar(p.dg, b * p.sdg[0] + t * p.sdg[1] + h * p.sdg[2], p.g_dtype, sg);
      store_scalar(p.dbeta, b * p.sdb[0] + t * p.sdb[1] + h * p.sdb[2], p.beta_dtype, sb);
    }
  }
}

// Workspace layout (floats, each part 256-byte aligned).
struct Layout {
  int64_t ckpt, pq, pk, pg, pb, total;  // offsets in bytes
  int64_t R, nslot;
};

inline int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

inline Layout layout(int B, int T, int H, int K, int V, int n_seq) {
  Layout L;
  const int64_t nv = V / BV, nch = (T + C - 1) / C;
  L.R = n_seq > 0 ? (int64_t)T : (int64_t)B * T;
  L.nslot = n_seq > 0 ? nch + n_seq : (int64_t)B * nch;
  int64_t off = 0;
  L.ckpt = off;
  off = align256(off + L.nslot * H * nv * K * BV * 4);
  L.pq = off;
  off = align256(off + nv * L.R * H * K * 4);
  L.pk = off;
  off = align256(off + nv * L.R * H * K * 4);
  L.pg = off;
  off = align256(off + nv * L.R * H * 4);
  L.pb = off;
  off = align256(off + nv * L.R * H * 4);
  L.total = off;
  return L;
}

template <typename TIn>
int launch_t(const BArgs& a, const RArgs& r, int K, int grid, hipStream_t s) {
  switch (K) {
    case 32: hipLaunchKernelGGL((bwd_kernel<TIn, 32>), dim3(grid), dim3(NT), 0, s, a); break;
    case 64: hipLaunchKernelGGL((bwd_kernel<TIn, 64>), dim3(grid), dim3(NT), 0, s, a); break;
    case 128: hipLaunchKernelGGL((bwd_kernel<TIn, 128>), dim3(grid), dim3(NT), 0, s, a); break;
    default: return GDN_ERR_UNSUPPORTED;
  }
  int err = (int)hipGetLastError();
  if (err != 0) return err;
  const int64_t work = r.R * r.H * (r.K + 1);
  const int rgrid = (int)std::min<int64_t>((work + 255) / 256, 4096);
  if (rgrid > 0) hipLaunchKernelGGL((reduce_kernel<TIn>), dim3(rgrid), dim3(256), 0, s, r);
  return (int)hipGetLastError();
}

}  // namespace bwd
}  // namespace gdn

using namespace gdn;

extern "C" int64_t gdn_bwd_workspace_size(int B, int T, int H, int K, int V, int n_seq) {
  if (B <= 0 || T < 0 || H <= 0 || V <= 0 || V % bwd::BV != 0 || n_seq < 0) return -1;
  if (K != 32 && K != 64 && K != 128) return -1;
  return bwd::layout(B, T, H, K, V, n_seq).total;
}

extern "C" int gdn_bwd_launch(const GdnBwdParams* prm, void* stream) {
  if (prm == nullptr) return GDN_ERR_NULL_POINTER;
  const GdnBwdParams& P = *prm;
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
  const int64_t units = (int64_t)P.B * P.H * (P.V / bwd::BV);
  if (units > 0x7fffffffLL || (int64_t)P.B * P.T * P.H * P.K >= (1LL << 40)) return GDN_ERR_BAD_SHAPE;
  // B is the number of sequences when cu_seqlens is given (one packed batch)
  const bwd::Layout L = bwd::layout(P.B, P.T, P.H, P.K, P.V, P.cu_seqlens ? P.B : 0);
  if (P.workspace == nullptr || reinterpret_cast<uintptr_t>(P.workspace) % 256 != 0 ||
      P.workspace_bytes < L.total)
    return GDN_ERR_WORKSPACE;
  if (P.T == 0 && P.dh0 == nullptr) return GDN_OK;

  char* ws = static_cast<char*>(P.workspace);
  bwd::BArgs a = {};
  a.q = P.q; a.k = P.k; a.v = P.v; a.g = P.g; a.beta = P.beta; a.h0 = P.h0;
  a.d_o = P.d_o; a.dfs = P.d_final_state; a.dv = P.dv; a.dh0 = P.dh0;
  a.ckpt = reinterpret_cast<float*>(ws + L.ckpt);
  a.pq = reinterpret_cast<float*>(ws + L.pq);
  a.pk = reinterpret_cast<float*>(ws + L.pk);
  a.pg = reinterpret_cast<float*>(ws + L.pg);
  a.pb = reinterpret_cast<float*>(ws + L.pb);
  for (int d = 0; d < 3; ++d) {
    a.sq[d] = P.q_stride[d]; a.sk[d] = P.k_stride[d]; a.sv[d] = P.v_stride[d];
    a.sg[d] = P.g_stride[d]; a.sb[d] = P.beta_stride[d]; a.sdo[d] = P.do_stride[d];
    a.sdv[d] = P.dv_stride[d];
  }
  for (int d = 0; d < 4; ++d) {
    a.sh0[d] = P.h0_stride[d]; a.sdfs[d] = P.dfs_stride[d]; a.sdh0[d] = P.dh0_stride[d];
  }
  a.R = L.R;
  a.B = P.B; a.T = P.T; a.H = P.H; a.V = P.V; a.nv = P.V / bwd::BV;
  a.scale = P.scale;
  a.g_dtype = P.g_dtype; a.beta_dtype = P.beta_dtype; a.do_dtype = P.do_dtype;
  a.cu = P.cu_seqlens;
  a.xcd_remap = (units % 8 == 0) ? 1 : 0;

  bwd::RArgs r = {};
  r.pq = a.pq; r.pk = a.pk; r.pg = a.pg; r.pb = a.pb;
  r.dq = P.dq; r.dk = P.dk; r.dg = P.dg; r.dbeta = P.dbeta;
  for (int d = 0; d < 3; ++d) {
    r.sdq[d] = P.dq_stride[d]; r.sdk[d] = P.dk_stride[d]; r.sdg[d] = P.dg_stride[d];
    r.sdb[d] = P.dbeta_stride[d];
  }
  r.R = P.T > 0 ? L.R : 0;
  r.T = P.T > 0 ? P.T : 1; r.H = P.H; r.K = P.K; r.nv = a.nv;
  r.qkv_dtype = P.qkv_dtype; r.g_dtype = P.g_dtype; r.beta_dtype = P.beta_dtype;

  hipStream_t s = static_cast<hipStream_t>(stream);
  const int grid = (int)units;
  switch (P.qkv_dtype) {
    case GDN_DTYPE_F16: return bwd::launch_t<f16>(a, r, P.K, grid, s);
    case GDN_DTYPE_BF16: return bwd::launch_t<bf16_t>(a, r, P.K, grid, s);
    default: return bwd::launch_t<float>(a, r, P.K, grid, s);
  }
}
