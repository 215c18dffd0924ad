// The forward for 32-row chunks as two launches: a per-chunk record of the
// state-independent work, then a scan over the chunks that keeps the state
// on chip (the default path for fp16 and bf16 inputs, C = 32, K in {64,
// 128}).
//
// Per chunk (C = 32 rows, b = in-chunk cumsum of g, as in gdn_ref.py:51-99):
//   A  = tril_-1(beta_t e^{b_t - b_j} K K^T),   T = (I + A)^-1,
//   Tu = T diag(beta),
//   u  = Tu (V - diag(e^b) K S)             (= U - W h^T, gdn_triton.py:87)
//   o  = scale (P u + diag(e^b) Q S),  P = tril_0(e^{b_t - b_j} Q K^T)
//   S' = e^{bC} S + K^T diag(e^{bC - b}) u  (the reference's h(e^{bC} I -
//        Wbar^T K) + Ubar^T K, gdn_ref.py:93-98, without the K x K temporary)
// Only u, o and S' involve the carried state.  A V-slice workgroup of the
// fused kernel would rebuild A and rerun the 32-row substitution for T once
// per slice; here they run once per (chunk, head):
//
//   1. rec32_kernel, one wave per two (chunk, head) records: K K^T on the
//      matrix cores, A, then T by forward substitution on the VALU (one lane
//      per row of T, rows of A^T broadcast from LDS), written with the gates
//      to a 3 KB record: Tu as MFMA operand fragments, b, e^b, e^{bC - b},
//      e^{bC}.
//   2. scan32_kernel, one workgroup per (sequence, head, BV-column slice),
//      walks the chunks with the fp32 K x BV state in accumulator registers
//      (no chunk state is written).  Waves have fixed roles and pass one
//      barrier per iteration:
//        SCAN x BV/16  chunk it: K S, Y = V - diag(e^b) K S, u = Tu Y,
//                      S <- e^{bC} S + K^T diag(e^{bC-b}) u (16 columns each;
//                      fp16 at BV = 16, K = 128: two waves, each updating
//                      half of the state rows)
//        OUT  x BV/16  chunk it: Q S with the chunk-start state;
//                      chunk it-1: o = scale (P u + diag(e^b) Q S), formed
//                      transposed so that each lane stores 8 consecutive
//                      elements of one row
//        PQK           chunk it: P = e^{b_t-b_j} Q K^T (t >= j) as hi + lo
//                      fp16 operand fragments
//        LOAD          chunk it+D: q, k, the v slice and the record, copied
//                      global -> LDS by the asynchronous LDS-DMA loads
//                      (global_load_lds_dwordx4), D chunks ahead.
//
// The records of a segment of L chunks per (sequence, head) live in the
// caller's workspace; a sequence longer than L chunks runs as several
// (rec32, scan32) pairs, the state passing from one segment to the next
// through final_state.  The workspace is therefore bounded by B * H * L
// records, independent of T.
//
// MFMA operand layouts, the state's key order and the transposing LDS reads
// are those of gdn_fwd_pipe.h (v_mfma_f32_16x16x32_f16; pi(g, s) pairing
// of accumulator rows and contraction slots).

#include "gdn_fwd_pipe.h"

namespace gdn {
namespace s32 {

using namespace pipe;

constexpr int C = 32;
constexpr int D = 4;  // chunks loaded ahead by the LOAD wave
constexpr int REC_BYTES = 3072;
// record layout (byte offsets)
constexpr int R_TU = 0;     // f16x8 [2][64]: Tu rows 16 mt + (lane & 15), columns pi(lane >> 4, s)
constexpr int R_B = 2048;   // float [32]: in-chunk cumsum b times log2(e) (flat past the sequence end)
constexpr int R_EB = 2176;  // float [32]: e^b
constexpr int R_EC = 2304;  // float [32]: e^{bC - b}
constexpr int R_EBC = 2432; // float: e^{bC}
// bf16 inputs: the record is followed by the chunk's k rows in fp16 (C x K,
// in frag_piece order, rows past the end holding the last row), which the
// scan copies instead of the input.
template <typename TIn, int K>
constexpr int rec_stride() {
  return std::is_same<TIn, bf16_t>::value ? REC_BYTES + C * K * 2 : REC_BYTES;
}
constexpr int R_K16 = REC_BYTES;
// 16-byte piece c (columns 8 c ..) of row r of those copies, in the order
// the record kernel's lanes hold them (lane (n, gq) of operand (mt, kb) is
// row 16 mt + n, piece 4 kb + gq): each of its stores is 1 KB contiguous.
template <int K>
__device__ __forceinline__ int frag_piece(int r, int c) {
  return ((((r >> 4) * (K / 32) + (c >> 2)) * 4 + (c & 3)) << 4) + (r & 15);
}

struct SArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  const float* h0;
  void* o;
  float* fs;
  char* rec;
  int64_t sq[3], sk[3], sv[3], sg[3], sb[3], so[3];
  int64_t sh0[4], sfs[4];
  int B, T, H, V, nv;  // B: sequences (units of row_span)
  int c0, L;           // this segment: chunks [c0, c0 + L) of every sequence
  int first;           // initial state from h0 (or zero) rather than final_state
  int nrec;            // B * H * L
  float scale;
  int g_dtype, beta_dtype, o_dtype;
  const int64_t* cu;
  int xcd_remap;
  int o_vec;           // o takes 16-byte stores (base and strides aligned for them)
};

// One barrier of the workgroup.  Written out (rather than __syncthreads)
// so that the LOAD wave's LDS-DMA copies in flight are not drained at every
// barrier: LDS writes of the issuing wave are complete (lgkmcnt), and the
// LOAD wave waits for the DMA copies it publishes itself.  The "memory"
// clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void wg_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt not waited for).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

typedef __attribute__((address_space(3))) void* lds_ptr;

// The fp16 rounding residual of two accumulator tiles given their fp16
// rounding h: lo = (f16)(x - (float)h), as split_lo, but written as
// fma(h, -one, x) so that each element is one v_fma_mix (h read as fp16
// from its half of the packed register, the result rounded to fp16).  x - h
// is exact in fp32, so the rounding is the same.  `one` is 1.0 held in a
// register the compiler cannot see through (opaque_one); with a literal 1
// the product is folded into a subtraction and the conversions return.
__device__ __forceinline__ float opaque_one() {
  float one = 1.0f;
  asm volatile("" : "+v"(one));
  return one;
}
__device__ __forceinline__ f16x8 split_lo_mix(const f32x4& lo, const f32x4& hi, const f16x8& h, float one) {
  return f16x8{(f16)__builtin_fmaf((float)h[0], -one, lo[0]), (f16)__builtin_fmaf((float)h[1], -one, lo[1]),
               (f16)__builtin_fmaf((float)h[2], -one, lo[2]), (f16)__builtin_fmaf((float)h[3], -one, lo[3]),
               (f16)__builtin_fmaf((float)h[4], -one, hi[0]), (f16)__builtin_fmaf((float)h[5], -one, hi[1]),
               (f16)__builtin_fmaf((float)h[6], -one, hi[2]), (f16)__builtin_fmaf((float)h[7], -one, hi[3])};
}

// 16 bytes per lane from global memory into LDS at base + 16 * lane.
__device__ __forceinline__ void dma16(const void* src, void* lds_base) {
  __builtin_amdgcn_global_load_lds(src, (lds_ptr)lds_base, 16, 0, 0);
}

// ---------------------------------------------------------------------------
// Phase stamps.  Built only with -DGDN_PHASE_STAMPS (build.py --phase-stamps,
// a separate library used by bench.py --phase-stamps): each MFMA phase is
// bracketed by s_memtime stamps, the first taken once the phase's operands
// are in registers (the stamp waits for outstanding LDS loads), the second
// once its results are, and the windows are summed per wave.  Dividing the
// phase's MFMA count times the measured cycles of one MFMA by the window
// gives the MFMA utilisation of the contraction phases on the SIMDs that
// run them.  The product library compiles none of this.
// ---------------------------------------------------------------------------

#ifdef GDN_PHASE_STAMPS
constexpr int PS_SLOTS = 8;                // counters per (workgroup, wave)
constexpr int PS_WG = 1024, PS_WAVES = 8;  // scan workgroups and waves recorded
constexpr int PS_REC = 16384;              // record-kernel waves recorded
__device__ unsigned long long g_phase_scan[PS_WG * PS_WAVES * PS_SLOTS];
__device__ unsigned long long g_phase_rec[PS_REC * 4];

// s_memtime once the given registers hold their values; the asm also
// "modifies" them, so no consumer is moved above the stamp.
template <typename A>
__device__ __forceinline__ unsigned long long ps_stamp(A& a) {
  unsigned long long t;
  asm volatile("s_memtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t), "+v"(a) :: "memory");
  return t;
}
template <typename A, typename B>
__device__ __forceinline__ unsigned long long ps_stamp(A& a, B& b) {
  unsigned long long t;
  asm volatile("s_memtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t), "+v"(a), "+v"(b) :: "memory");
  return t;
}
template <typename A, typename B, typename Cc>
__device__ __forceinline__ unsigned long long ps_stamp(A& a, B& b, Cc& c) {
  unsigned long long t;
  asm volatile("s_memtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t), "+v"(a), "+v"(b), "+v"(c) :: "memory");
  return t;
}
template <typename A, typename B, typename Cc, typename Dd>
__device__ __forceinline__ unsigned long long ps_stamp(A& a, B& b, Cc& c, Dd& d) {
  unsigned long long t;
  asm volatile("s_memtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t), "+v"(a), "+v"(b), "+v"(c), "+v"(d) :: "memory");
  return t;
}
// slots of (workgroup, wave): role, chunks, window A, window B, MFMAs per
// window A, per window B
__device__ __forceinline__ void ps_record(int wave, int lane, unsigned long long role, unsigned long long n,
                                          unsigned long long wa, unsigned long long wb, unsigned long long ma,
                                          unsigned long long mb) {
  if (lane == 0 && blockIdx.x < PS_WG && wave < PS_WAVES) {
    unsigned long long* d = g_phase_scan + ((int64_t)blockIdx.x * PS_WAVES + wave) * PS_SLOTS;
    d[0] = role; d[1] = n; d[2] = wa; d[3] = wb; d[4] = ma; d[5] = mb;
  }
}
// slots 6 and 7: the cycles this wave spent in its barriers (from just
// before the LDS drain that precedes each s_barrier to its release) and the
// cycles from its first barrier's release to the end of its chunk loop
__device__ __forceinline__ void ps_record_bar(int wave, int lane, unsigned long long role, unsigned long long n,
                                              unsigned long long bar, unsigned long long loop) {
  if (lane == 0 && blockIdx.x < PS_WG && wave < PS_WAVES) {
    unsigned long long* d = g_phase_scan + ((int64_t)blockIdx.x * PS_WAVES + wave) * PS_SLOTS;
    d[0] = role; d[1] = n; d[6] = bar; d[7] = loop;
  }
}
__device__ __forceinline__ unsigned long long ps_now() {
  unsigned long long t;
  asm volatile("s_memtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(t) :: "memory");
  return t;
}
#define PS_DECL unsigned long long ps_a = 0, ps_b = 0, ps_t0 = 0
#define PS_BEGIN(...) ps_t0 = ps_stamp(__VA_ARGS__)
#define PS_END_A(...) ps_a += ps_stamp(__VA_ARGS__) - ps_t0
#define PS_END_B(...) ps_b += ps_stamp(__VA_ARGS__) - ps_t0
#define PS_RECORD(role, n, ma, mb) ps_record(wave, lane, role, n, ps_a, ps_b, ma, mb)
#else
#define PS_DECL
#define PS_BEGIN(...)
#define PS_END_A(...)
#define PS_END_B(...)
#define PS_RECORD(role, n, ma, mb)
#endif

// ---------------------------------------------------------------------------
// 1. records
// ---------------------------------------------------------------------------

// Record r of a segment is (sequence bi, head hi, chunk c0 + lc) with
// r = (bi * H + hi) * L + lc.
__device__ __forceinline__ void rec_coords(const SArgs& p, int r, int& bi, int& hi, int& lc) {
  lc = r % p.L;
  const int bh = r / p.L;
  hi = bh % p.H;
  bi = bh / p.H;
}

template <typename TIn, int K>
__global__ __launch_bounds__(256) void rec32_kernel(const SArgs p) {
  constexpr int KB = K / 32;
  constexpr uint32_t EB = sizeof(TIn);
  // per wave and record: A^T row-major (at[j][t] = A[t][j]), beta and b
  __shared__ __attribute__((aligned(16))) float s_at[4][2][C * C];
  __shared__ __attribute__((aligned(16))) float s_beta[4][2][C];
  __shared__ __attribute__((aligned(16))) float s_b[4][2][C];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, gq = lane >> 4;
  const int half = lane >> 5, c = lane & 31;
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};

  // the two records of this wave: geometry (wave-uniform)
  int nval[2];
  const char* kh[2];
  char* rp[2];
  uint32_t skb[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int r = (blockIdx.x * 4 + wave) * 2 + e;
    nval[e] = 0;
    kh[e] = nullptr;
    rp[e] = nullptr;
    skb[e] = 0;
    if (r < p.nrec) {
      int bi, hi, lc;
      rec_coords(p, r, bi, hi, lc);
      const RowSpan rs = row_span(p.cu, p.T, bi);
      const int t0 = (p.c0 + lc) * C;
      if (t0 < rs.T) {
        nval[e] = min(C, rs.T - t0);
        kh[e] = static_cast<const char*>(p.k) + (head_base(rs, hi, p.sk) + (int64_t)t0 * p.sk[1]) * EB;
        skb[e] = (uint32_t)p.sk[1] * EB;
        rp[e] = p.rec + (int64_t)r * rec_stride<TIn, K>();
      }
    }
  }
  // k rows (rows past the end re-read the last row: finite values whose
  // beta is zero), then the gates of row c of record `half`
  uint4 kr[2][2][KB];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    if (nval[e] > 0) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const int rr = min(16 * mt + n, nval[e] - 1);
          kr[e][mt][kb] = ld16(kh[e], (uint32_t)rr * skb[e] + (32 * kb + 8 * gq) * EB);
        }
    }
  }
  float gv = 0.f, bv = 0.f;
  {
    const int e = half;
    const int r = (blockIdx.x * 4 + wave) * 2 + e;
    if (r < p.nrec && c < nval[e]) {
      int bi, hi, lc;
      rec_coords(p, r, bi, hi, lc);
      const RowSpan rs = row_span(p.cu, p.T, bi);
      const int64_t t = (int64_t)(p.c0 + lc) * C + c;
      gv = load_scalar(p.g, head_base(rs, hi, p.sg) + t * p.sg[1], p.g_dtype);
      bv = load_scalar(p.beta, head_base(rs, hi, p.sb) + t * p.sb[1], p.beta_dtype);
    }
  }
  // gates (lanes 0-31: record 0, lanes 32-63: record 1)
  const float b = scan32(gv);
  const float bC0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(b), 31));
  const float bC1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(b), 63));
  const float bC = half ? bC1 : bC0;
  s_beta[wave][half][c] = bv;
  s_b[wave][half][c] = b;
  if (nval[half] > 0) {
    char* rr = rp[half];
    reinterpret_cast<float*>(rr + R_B)[c] = b * 1.4426950408889634f;
    reinterpret_cast<float*>(rr + R_EB)[c] = fexp(b);
    reinterpret_cast<float*>(rr + R_EC)[c] = fexp(bC - b);
    if (c == 0) *reinterpret_cast<float*>(rr + R_EBC) = fexp(bC);
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

  // A = beta_t e^{b_t - b_j} K K^T (t > j), stored as A^T
#ifdef GDN_PHASE_STAMPS
  unsigned long long ps_r0 = ps_stamp(kr[0][0][0].x, kr[1][0][0].x);
  int ps_n = 0;
#endif
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    if (nval[e] > 0) {
#ifdef GDN_PHASE_STAMPS
      ps_n += 3 * KB;
#endif
      f16x8 kf[2][KB];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) kf[mt][kb] = to_f16x8<TIn>(kr[e][mt][kb]);
      if constexpr (std::is_same<TIn, bf16_t>::value) {
        // the k rows in fp16 after the record (lane (n, gq): rows 16 mt + n,
        // columns 32 kb + 8 gq ..; rows past the end repeat the last row)
        f16* const k16 = reinterpret_cast<f16*>(rp[e] + R_K16);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
            *reinterpret_cast<f16x8*>(k16 + 8 * frag_piece<K>(16 * mt + n, 4 * kb + gq)) = kf[mt][kb];
      }
      float* sa = s_at[wave][e];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt <= mt; ++nt) {
          f32x4 acc = z4;
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) acc = Mma<f16>::mma(kf[mt][kb], kf[nt][kb], acc);
          const int jj = 16 * nt + n;
          const float bj = s_b[wave][e][jj];
          const f32x4 bt4 = *reinterpret_cast<const f32x4*>(&s_b[wave][e][16 * mt + 4 * gq]);
          const f32x4 be4 = *reinterpret_cast<const f32x4*>(&s_beta[wave][e][16 * mt + 4 * gq]);
          f32x4 av;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int t = 16 * mt + 4 * gq + i;
            const float x = t > jj ? bt4[i] - bj : -__builtin_inff();
            av[i] = acc[i] * fexp(x) * be4[i];
          }
          *reinterpret_cast<f32x4*>(sa + jj * C + 16 * mt + 4 * gq) = av;
        }
    }
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#ifdef GDN_PHASE_STAMPS
  {
    unsigned long long ps_r1;
    asm volatile("s_memtime %0\n\ts_waitcnt lgkmcnt(0)" : "=s"(ps_r1) :: "memory");
    const int w = blockIdx.x * 4 + wave;
    if (lane == 0 && w < PS_REC) {
      g_phase_rec[4 * w] = 1;
      g_phase_rec[4 * w + 1] = ps_r1 - ps_r0;
      g_phase_rec[4 * w + 2] = ps_n;
    }
  }
#endif

  // T by substitution: lane c of half h holds row c of T of record h
  float xc[C];
#pragma unroll
  for (int i = 0; i < C; ++i) xc[i] = 0.f;
  const float* at = s_at[wave][half];
  solve_rows<19, 32>(at, c, xc);
  solve_rows<13, 19>(at, c, xc);
  solve_rows<9, 13>(at, c, xc);
  solve_rows1<6, 9>(at, c, xc);
  solve_rows1<3, 6>(at, c, xc);
  solve_rows1<0, 3>(at, c, xc);
  if (nval[half] > 0) {
    // row c of Tu = T diag(beta): operand tile c / 16, lane (c % 16, g4)
    const float* bt = s_beta[wave][half];
    f16x8* tu = reinterpret_cast<f16x8*>(rp[half] + R_TU);
    const int mt = c >> 4, nl = c & 15;
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const f32x4 u0 = *reinterpret_cast<const f32x4*>(&bt[4 * g4]);
      const f32x4 u1 = *reinterpret_cast<const f32x4*>(&bt[16 + 4 * g4]);
      f16x8 fu;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        fu[e] = (f16)(xc[4 * g4 + e] * u0[e]);
        fu[4 + e] = (f16)(xc[16 + 4 * g4 + e] * u1[e]);
      }
      tu[mt * 64 + 16 * g4 + nl] = fu;
    }
  }
}

// ---------------------------------------------------------------------------
// 2. the scan
// ---------------------------------------------------------------------------

template <int K, int BV>
struct alignas(16) ScanSmem {
  static constexpr int NSW = BV / 16;
  static constexpr int R = D + 1;   // q, k, v slots: read in the chunk's own iteration
  static constexpr int RR = D + 2;  // record slots: e^b is read once more by OUT
  f16x8 rq[R][C][K / 8];            // q rows, 16-byte piece c of row r at swz(r, c)
  f16x8 rk[R][C][K / 8];            // k rows, likewise
  f16x8 rv[R][C][BV / 8];           // v slice rows (plain)
  char rec[RR][REC_BYTES];
  f16x8 p[2][2][64];                // P operand fragments, hi
  f16x8 plo[2][2][64];              // and the fp16 residual
  f16x8 so[2][NSW][K / 32][64];     // chunk-start state as B operand fragments
  f32x4 uo[2][NSW][2][64];          // u in fp32 (accumulator layout)
  float usc[2][NSW][2];             // bf16: u's range factors for OUT (Q S ratio, o scale)
};

// bf16 inputs: the range shift of a 16-column state slice, chosen chunk by
// chunk.  Each SCAN wave runs its columns on v and the state times 2^sh, a
// power of two (exact in fp32, and carried unchanged through fp16 rounding
// away from fp16's limits), and o and final_state come out times 2^-sh.
// The shift only goes down along the sequence: sh_c = min(sh_{c-1},
// cap(chunk c's v)), starting from cap(incoming state), so that every
// operand already folded into the state stays in range; going down, the
// state is multiplied by 2^(sh_c - sh_{c-1}) with the chunk's decay.  o and
// the state are linear in (v, state) and each column evolves on its own,
// which makes this exact up to the roundings the unscaled values would see.
// cap(m), for a largest magnitude with float bits m (wave-uniform): none
// (kNoCap) when m is zero, 0 when m is not finite or lies in [2^-6, 2^10],
// else 127 - e for m's biased exponent e, which puts m 2^cap in [1, 2);
// clamped to [-126, 126].
constexpr int kNoCap = 127;
__device__ __forceinline__ int shift_cap(uint32_t m) {
  if (m == 0) return kNoCap;
  const int e = (int)(m >> 23);
  if (e >= 255 || (m >= 0x3c800000u && m <= 0x44800000u)) return 0;
  return min(max(127 - e, -126), 126);
}

// 2^n for n in [-126, 127], built from its bits (scalar for uniform n).
__device__ __forceinline__ float pow2i(int n) { return __int_as_float((n + 127) << 23); }

// Largest of m over the wave (as unsigned), wave-uniform: DPP within rows
// of 16 lanes, then the four row results.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t m) {
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0xb1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x4e, 0xf, 0xf, false));   // quad_perm 2,3,0,1
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x141, 0xf, 0xf, false));  // row_half_mirror
  m = max(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x140, 0xf, 0xf, false));  // row_mirror
  const uint32_t a = __builtin_amdgcn_readlane(m, 0), b = __builtin_amdgcn_readlane(m, 16);
  const uint32_t c = __builtin_amdgcn_readlane(m, 32), d = __builtin_amdgcn_readlane(m, 48);
  return max(max(a, b), max(c, d));
}

// Whether the largest of m over the lanes set in `lanes` (m: float bits
// of magnitudes) lies in [2^-6, 2^10], where shift_cap is 0: two compares,
// no cross-lane reduction (the usual case).
__device__ __forceinline__ bool cap0_lanes(uint32_t m, uint64_t lanes) {
  const uint64_t big = __builtin_amdgcn_ballot_w64(m > 0x44800000u) & lanes;
  const uint64_t mid = __builtin_amdgcn_ballot_w64(m >= 0x3c800000u) & lanes;
  return big == 0 && mid != 0;
}

// shift_cap of the largest of m over the wave.
__device__ __forceinline__ int wave_cap(uint32_t m) {
  return cap0_lanes(m, ~0ull) ? 0 : shift_cap(wave_max_u32(m));
}

// A 16-bit element holding bf16 bits: its value, and |value| as fp32 bits.
__device__ __forceinline__ float bf16_bits_f32(f16 x) {
  return __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, x) << 16);
}
__device__ __forceinline__ uint32_t bf16_abs_bits(f16 x) {
  return ((uint32_t)__builtin_bit_cast(uint16_t, x) & 0x7fffu) << 16;
}

// Two floats as packed fp16 (round to nearest even, as (f16) x).
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  typedef f16 f16x2v __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, f16x2v{(f16)a, (f16)b});
}

// 4 consecutive o elements at o + off: one 16-byte store (fp32 o, when
// `vec`: base and strides aligned for it), else one store per element.
template <typename TOut>
__device__ __forceinline__ void store_o4(void* o, int64_t off, const f32x4& w, int vec) {
  if (vec) {
    if constexpr (std::is_same<TOut, f16>::value) {
      typedef f16 f16x4v __attribute__((ext_vector_type(4)));
      *reinterpret_cast<f16x4v*>(static_cast<f16*>(o) + off) = f16x4v{(f16)w[0], (f16)w[1], (f16)w[2], (f16)w[3]};
    } else if constexpr (std::is_same<TOut, bf16_t>::value) {
      auto pk = [](float a, float b) { return (uint32_t)float_to_bf16_bits(a) | ((uint32_t)float_to_bf16_bits(b) << 16); };
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(o) + off) = uint2{pk(w[0], w[1]), pk(w[2], w[3])};
    } else {
      *reinterpret_cast<f32x4*>(static_cast<float*>(o) + off) = w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) put<TOut>(o, off + i, w[i]);
  }
}

// fp16 at BV = 16 and K = 128 can split the slice's SCAN work over two
// waves, each updating half of the state rows (five waves): SCAN is the
// longest role there.  The launch takes the split for segments of at most
// kSplitChunks chunks; longer ones run faster on one SCAN wave, and at
// K = 64 the split costs more than it saves.
template <typename TIn, int K, int BV>
constexpr bool scan_split_ok() {
  return std::is_same<TIn, f16>::value && BV == 16 && K == 128;
}
constexpr int kSplitChunks = 192;

template <int BV, bool SPL>
constexpr int scan_waves() {
  return 2 * (BV / 16) + 2 + (SPL ? 1 : 0);
}

enum ScanRole { SR_SCAN, SR_OUT, SR_PQK, SR_LOAD };

// DMA copies per chunk: q and k (1 KB each), the v slice, the record.
template <int K, int BV>
constexpr int dma_per_chunk() {
  return 2 * (C * K * 2 / 1024) + (C * BV * 2 + 1023) / 1024 + REC_BYTES / 1024;
}

template <typename TIn, int K, int BV, bool SPLIT>
__global__ __launch_bounds__((64 * scan_waves<BV, SPLIT>())) void scan32_kernel(const SArgs p) {
  using M = Mma<f16>;
  using S = ScanSmem<K, BV>;
  constexpr int NSW = BV / 16;
  static_assert(!SPLIT || scan_split_ok<TIn, K, BV>(), "split SCAN: fp16, K = 128, BV = 16");
  constexpr int KB = K / 32, KT = K / 16;
  constexpr int R = S::R, RR = S::RR;
  constexpr int ND = dma_per_chunk<K, BV>();
  static_assert(sizeof(TIn) == 2, "16-bit inputs");
  static_assert(std::is_same<TIn, f16>::value || std::is_same<TIn, bf16_t>::value, "fp16 or bf16 inputs");
  static_assert((D - 2) * ND < 64, "outstanding DMA copies fit vmcnt");
  static_assert(C * BV * 2 % 1024 == 0, "v slice rows fill whole DMA copies");

  __shared__ S s;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
#ifdef GDN_PHASE_STAMPS
  // the workgroup barrier, timed (stamps build only): the time in each
  // barrier after the first, and the loop's cycles from the first
  // barrier's release
  unsigned long long ps_bar = 0, ps_loop0 = 0;
  int ps_nb = 0;
  auto wg_barrier = [&]() __attribute__((always_inline)) {
    const unsigned long long t0 = ps_now();
    s32::wg_barrier();
    const unsigned long long t1 = ps_now();
    if (ps_nb++ == 0)
      ps_loop0 = t1;
    else
      ps_bar += t1 - t0;
  };
#define PS_RECORD_BAR(role) ps_record_bar(wave, tid & 63, role, nloc, ps_bar, ps_now() - ps_loop0)
#else
#define PS_RECORD_BAR(role)
#endif
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
  const RowSpan rs = row_span(p.cu, p.T, bi);
  const int T = rs.T;
  const int nch_all = (T + C - 1) / C;
  const int nloc = max(0, min(p.L, nch_all - p.c0));  // chunks of this segment
  if (nloc == 0 && !p.first) return;                  // state unchanged
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};

  constexpr uint32_t EB = sizeof(TIn);
  const uint32_t sqb = (uint32_t)p.sq[1] * EB, skb = (uint32_t)p.sk[1] * EB;
  const uint32_t svb = (uint32_t)p.sv[1] * EB;
  const char* qh = static_cast<const char*>(p.q) + head_base(rs, hi, p.sq) * EB;
  const char* kh = static_cast<const char*>(p.k) + head_base(rs, hi, p.sk) * EB;
  const char* vh = static_cast<const char*>(p.v) + (head_base(rs, hi, p.sv) + v0) * EB;
  constexpr int RS = rec_stride<TIn, K>();
  const char* rech = p.rec + (int64_t)(bi * p.H + hi) * p.L * RS;
  // the incoming state: h0 (nullable) on the first segment, else the
  // previous segment's final state
  const float* const st_src = p.first ? p.h0 : p.fs;
  const int64_t* const st_sd = p.first ? p.sh0 : p.sfs;
  constexpr bool BF = std::is_same<TIn, bf16_t>::value;  // range shifts (shift_cap)

  auto staged = [&](const f16x8 (&tile)[C][K / 8], int r, int cc) { return tile[r][swz<K>(r, cc)]; };

  // Waves w and w + 4 share SIMD w % 4.  At BV = 32 (six waves) LOAD and
  // the second OUT wave are alone on their SIMDs; the first SCAN wave shares
  // its SIMD with PQK, the second with the first OUT wave, each the older
  // wave of its pair (of twelve placements timed: bf16 7-10 % faster than
  // with the SCAN waves alone and LOAD beside an OUT wave, fp16 the same).
  // Split SCAN (five waves): the two SCAN waves and PQK each alone on a
  // SIMD, OUT with LOAD (of the five placements timed, the fastest: a SCAN
  // or PQK wave beside LOAD or each other is slower).
  int role, ridx;
  if constexpr (SPLIT) {
    constexpr int roles[5] = {SR_OUT, SR_PQK, SR_SCAN, SR_SCAN, SR_LOAD};
    constexpr int idx[5] = {0, 0, 0, 1, 0};
    role = roles[wave];
    ridx = idx[wave];
  } else if constexpr (NSW == 2) {
    constexpr int roles[6] = {SR_SCAN, SR_OUT, SR_LOAD, SR_OUT, SR_PQK, SR_SCAN};
    constexpr int idx[6] = {0, 0, 0, 1, 0, 1};
    role = roles[wave];
    ridx = idx[wave];
  } else {
    role = wave == 0 ? SR_SCAN : wave == 1 ? SR_OUT : wave == 2 ? SR_PQK : SR_LOAD;
    ridx = 0;
  }

  if (role == SR_SCAN) {
    // ================================================================ SCAN
    // NH state waves per 16-column slice.  NH = 2 (fp16 at BV = 16): wave h
    // keeps the state rows of key blocks h KB / 2 .. (h + 1) KB / 2 - 1 and
    // updates them; both form the whole K S, reading the other half of S
    // from the chunk-start copy in LDS (written before the last barrier),
    // and the whole u.  NH = 1: one wave per slice (cb: the slice at BV = 32).
    auto scan = [&](auto HH, auto NHH) __attribute__((always_inline)) {
      constexpr int h = decltype(HH)::value, NH = decltype(NHH)::value;
      constexpr int KBO = KB / NH, KTO = KT / NH;  // own 32-key blocks, own 16-key state tiles
      constexpr int kb0 = h * KBO, r0 = h * KTO;
      constexpr int KBP = NH == 2 ? KB - KBO : 1;  // the other wave's blocks
      constexpr int kbp0 = (1 - h) * KBO;
      const int cb = NH == 1 ? ridx : 0;
      const float one = opaque_one();
      const int vcol = 16 * cb + n;
      // accumulator element (r, i) is state row rho = 16 r + 4 gq + i
      auto key_of = [&](int r, int i) { return 32 * (r >> 1) + 8 * gq + 4 * (r & 1) + i; };
      f32x4 st[KTO];
      {
        const float* src = st_src;
        const int64_t* sd = st_sd;
#pragma unroll
        for (int rl = 0; rl < KTO; ++rl) st[rl] = z4;
        if (src != nullptr) {
          const float* s0 = src + bi * sd[0] + hi * sd[1] + (v0 + vcol) * sd[3];
#pragma unroll
          for (int rl = 0; rl < KTO; ++rl)
#pragma unroll
            for (int i = 0; i < 4; ++i) st[rl][i] = s0[key_of(r0 + rl, i) * sd[2]];
        }
      }
      // bf16: the shift bound (sc) and the shift in use (sh), from the
      // incoming state's columns
      int sc = kNoCap, sh = 0;
      if constexpr (BF) {
        uint32_t m = 0;
#pragma unroll
        for (int rl = 0; rl < KTO; ++rl)
#pragma unroll
          for (int i = 0; i < 4; ++i) m = max(m, __float_as_uint(st[rl][i]) & 0x7fffffffu);
        sc = wave_cap(m);
        sh = sc == kNoCap ? 0 : sc;
        const float f = pow2i(sh);
#pragma unroll
        for (int rl = 0; rl < KTO; ++rl) st[rl] = st[rl] * f;
      }
      f16x8 sB[KBO];
#pragma unroll
      for (int kl = 0; kl < KBO; ++kl) {
        sB[kl] = M::from_acc(st[2 * kl], st[2 * kl + 1]);
        s.so[0][cb][kb0 + kl][lane] = sB[kl];
      }
      PS_DECL;
      // One chunk's operands of the chain, in registers.  Chunk it + 1's are
      // read from LDS while chunk it computes (the LOAD wave publishes chunks
      // two ahead), so the chain K S -> u -> S waits on no LDS read.
      struct ScanOps {
        f16x8 kR[2][KB], kA[KTO];
        f16x4 va, vb;
        f16x8 tu0, tu1;
        f32x4 eb_lo, eb_hi, ec_lo, ec_hi;
        float ebC;
      };
      // the cap of a chunk's v column from the operands in registers
      auto own_cap = [&](const ScanOps& x) __attribute__((always_inline)) {
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) m = max(m, max(bf16_abs_bits(x.va[i]), bf16_abs_bits(x.vb[i])));
        return wave_cap(m);
      };
      const int t0 = 4 * gq + (n >> 2), t1 = t0 + 16;
      const int vc = (16 * cb + 4 * (n & 3)) * 2;
      auto read_kA = [&](const char* kbase, int rl) __attribute__((always_inline)) {
        const int r = r0 + rl;
        const int piece = 4 * (r >> 1) + (n & 3);
        const f16x4 lo = lds_tr16(kbase + t0 * (K * 2) + swz<K>(t0, piece) * 16 + (r & 1) * 8);
        const f16x4 hi4 = lds_tr16(kbase + t1 * (K * 2) + swz<K>(t1, piece) * 16 + (r & 1) * 8);
        return cat8(lo, hi4);
      };
      // bf16: a chunk's shift from the cap of its v column, taken at the
      // chunk's start (the usual cap 0 costs two compares, off the K S
      // products' path); dsh is the change from the previous chunk's shift
      // (< 0, or > 0 only while the state is zero)
      int dsh = 0;
      auto take_cap = [&](int cap) __attribute__((always_inline)) {
        sc = min(sc, cap);
        const int shn = sc == kNoCap ? 0 : sc;
        dsh = shn - sh;
        sh = shn;
      };
      auto read_ops = [&](int it, ScanOps& o) __attribute__((always_inline)) {
        const int sl = it % R;
        const char* rc = s.rec[it % RR];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) o.kR[mt][kb] = staged(s.rk[sl], 16 * mt + n, 4 * kb + gq);
        const char* kbase = reinterpret_cast<const char*>(s.rk[sl]);
#pragma unroll
        for (int rl = 0; rl < KTO; ++rl) o.kA[rl] = read_kA(kbase, rl);
        // v rows 4 gq + i and 16 + 4 gq + i of column vcol (accumulator layout)
        const char* vbase = reinterpret_cast<const char*>(s.rv[sl]);
        o.va = lds_tr16(vbase + t0 * (BV * 2) + vc);
        o.vb = lds_tr16(vbase + t1 * (BV * 2) + vc);
        const f16x8* tu = reinterpret_cast<const f16x8*>(rc + R_TU);
        o.tu0 = tu[lane];
        o.tu1 = tu[64 + lane];
        const float* ebr = reinterpret_cast<const float*>(rc + R_EB);
        const float* ecr = reinterpret_cast<const float*>(rc + R_EC);
        o.eb_lo = *reinterpret_cast<const f32x4*>(ebr + 4 * gq);
        o.eb_hi = *reinterpret_cast<const f32x4*>(ebr + 16 + 4 * gq);
        o.ec_lo = *reinterpret_cast<const f32x4*>(ecr + 4 * gq);
        o.ec_hi = *reinterpret_cast<const f32x4*>(ecr + 16 + 4 * gq);
        o.ebC = *reinterpret_cast<const float*>(rc + R_EBC);
      };
      // The next chunk's reads go out between the chain's MFMAs (a few per
      // MFMA, placed by sched_group_barrier): issued all at once they would
      // fill the wave's LDS queue and hold the first MFMA back until most had
      // returned.
      constexpr int SG_VALU = 0x2, SG_MFMA = 0x8, SG_DSR = 0x100;
      auto chunk = [&](int it, ScanOps& o, ScanOps& nx) __attribute__((always_inline)) {
        const int itn = min(it + 1, nloc - 1);  // the last chunk's again at the end
        const int sl = itn % R;
        const char* rc = s.rec[itn % RR];
        // the other wave's half of this chunk's start state
        f16x8 sP[KBP];
        if constexpr (NH == 2) {
#pragma unroll
          for (int j = 0; j < KBP; ++j) sP[j] = s.so[it & 1][cb][kbp0 + j][lane];
        }
        // bf16: the state (and K S, Q S of the chunk-start state) change
        // units by 2^dsh
        float ebC = o.ebC, rat = 1.f, vmul = 1.f;
        if constexpr (BF) {
          take_cap(own_cap(o));
          rat = pow2i(max(dsh, -126));
          ebC = dsh >= -126 ? ebC * rat : ldexpf(ebC, dsh);
          vmul = pow2i(sh);
        }
        // K S: rows t, so its two row tiles form a B operand over t; own
        // key blocks first, the next chunk's k rows in between
        f32x4 ks[2] = {z4, z4};
        PS_BEGIN(o.kR[0][0], o.kR[1][0], sB[0], o.kA[0]);
        // e^{b_C} S, in place: the multiplies fill the VALU slots between
        // the K S products (sB already holds this chunk's S) instead of
        // delaying the state update at the end of the chain
#pragma unroll
        for (int rl = 0; rl < KTO; ++rl) st[rl] = st[rl] * ebC;
#pragma unroll
        for (int j = 0; j < KB; ++j) {
          const int kb = NH == 2 ? (j < KBO ? kb0 + j : kbp0 + j - KBO) : j;
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) {
            const f16x8 sop = (NH == 1 || j < KBO) ? sB[min(j, KBO - 1)] : sP[max(j - KBO, 0) % KBP];
            ks[mt] = M::mma(o.kR[mt][kb], sop, ks[mt]);
            nx.kR[mt][kb] = staged(s.rk[sl], 16 * mt + n, 4 * kb + gq);
          }
        }
#pragma unroll
        for (int g = 0; g < 2 * KB; ++g) {
          __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
          __builtin_amdgcn_sched_group_barrier(SG_DSR, 1, 0);
          __builtin_amdgcn_sched_group_barrier(SG_VALU, 4, 0);
        }
        f32x4 y0, y1;
        if constexpr (BF) {
          // v from its bf16 bits, times 2^sh (the multiplies only where a
          // shift is in use)
          if (sh == 0 && dsh == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              y0[i] = bf16_bits_f32(o.va[i]) - o.eb_lo[i] * ks[0][i];
              y1[i] = bf16_bits_f32(o.vb[i]) - o.eb_hi[i] * ks[1][i];
            }
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              y0[i] = bf16_bits_f32(o.va[i]) * vmul - (o.eb_lo[i] * rat) * ks[0][i];
              y1[i] = bf16_bits_f32(o.vb[i]) * vmul - (o.eb_hi[i] * rat) * ks[1][i];
            }
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            y0[i] = (float)o.va[i] - o.eb_lo[i] * ks[0][i];
            y1[i] = (float)o.vb[i] - o.eb_hi[i] * ks[1][i];
          }
        }
        const f16x8 yB = M::from_acc(y0, y1);
        f32x4 u[2];
        u[0] = M::mma(o.tu0, yB, z4);
        u[1] = M::mma(o.tu1, yB, z4);
        {
          // the next chunk's v column and record fields
          const char* vbase = reinterpret_cast<const char*>(s.rv[sl]);
          nx.va = lds_tr16(vbase + t0 * (BV * 2) + vc);
          nx.vb = lds_tr16(vbase + t1 * (BV * 2) + vc);
          const f16x8* tu = reinterpret_cast<const f16x8*>(rc + R_TU);
          nx.tu0 = tu[lane];
          nx.tu1 = tu[64 + lane];
          const float* ebr = reinterpret_cast<const float*>(rc + R_EB);
          const float* ecr = reinterpret_cast<const float*>(rc + R_EC);
          nx.eb_lo = *reinterpret_cast<const f32x4*>(ebr + 4 * gq);
          nx.eb_hi = *reinterpret_cast<const f32x4*>(ebr + 16 + 4 * gq);
          nx.ec_lo = *reinterpret_cast<const f32x4*>(ecr + 4 * gq);
          nx.ec_hi = *reinterpret_cast<const f32x4*>(ecr + 16 + 4 * gq);
          nx.ebC = *reinterpret_cast<const float*>(rc + R_EBC);
        }
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
        __builtin_amdgcn_sched_group_barrier(SG_DSR, 5, 0);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
        __builtin_amdgcn_sched_group_barrier(SG_DSR, 4, 0);
        const f16x8 utB = M::from_acc(u[0] * o.ec_lo, u[1] * o.ec_hi);
        // state update of the own rows; the next chunk's transposed k
        // fragments in between
        const char* kbase = reinterpret_cast<const char*>(s.rk[sl]);
#pragma unroll
        for (int rl = 0; rl < KTO; ++rl) {
          st[rl] = M::mma(o.kA[rl], utB, st[rl]);
          nx.kA[rl] = read_kA(kbase, rl);
        }
#pragma unroll
        for (int rl = 0; rl < KTO; ++rl) {
          __builtin_amdgcn_sched_group_barrier(SG_MFMA, 1, 0);
          __builtin_amdgcn_sched_group_barrier(SG_DSR, 2, 0);
        }
        if constexpr (NH == 2) {
          // u for OUT as fp16 hi and residual operand fragments, in the two
          // 16-byte slots of the fp32 copy, from wave 0 (wave 1 sums K S
          // in another order: its u may differ in the last fp32 bit, which
          // only its own state rows see)
          if (h == 0) {
            const f16x8 uhi = M::from_acc(u[0], u[1]);
            reinterpret_cast<f16x8*>(&s.uo[it & 1][cb][0][0])[lane] = uhi;
            reinterpret_cast<f16x8*>(&s.uo[it & 1][cb][1][0])[lane] = split_lo_mix(u[0], u[1], uhi, one);
          }
        } else {
          s.uo[it & 1][cb][0][lane] = u[0];
          s.uo[it & 1][cb][1][lane] = u[1];
          if constexpr (BF) {
            // OUT: Q S of the chunk-start state times rat, o times 2^-sh
            if (lane == 0) {
              s.usc[it & 1][cb][0] = rat;
              s.usc[it & 1][cb][1] = p.scale * pow2i(-sh);
            }
          }
        }
#pragma unroll
        for (int kl = 0; kl < KBO; ++kl) sB[kl] = M::from_acc(st[2 * kl], st[2 * kl + 1]);
        PS_END_A(sB[0], sB[KBO - 1]);
#pragma unroll
        for (int kl = 0; kl < KBO; ++kl) s.so[(it + 1) & 1][cb][kb0 + kl][lane] = sB[kl];
        wg_barrier();
      };
      ScanOps oa, ob;
      if (nloc > 0) {
        wg_barrier();
        read_ops(0, oa);
      }
      for (int it = 0; it < nloc; it += 2) {
        chunk(it, oa, ob);
        if (it + 1 < nloc) chunk(it + 1, ob, oa);
      }
      PS_RECORD(1, nloc, 2 * KB + 2 + KTO, 0);
      PS_RECORD_BAR(1);
      float* fs = p.fs + bi * p.sfs[0] + hi * p.sfs[1] + (v0 + vcol) * p.sfs[3];
      const float fsc = pow2i(-sh);
#pragma unroll
      for (int rl = 0; rl < KTO; ++rl)
#pragma unroll
        for (int i = 0; i < 4; ++i) fs[key_of(r0 + rl, i) * p.sfs[2]] = st[rl][i] * fsc;
    };
    if constexpr (SPLIT) {
      if (ridx == 0)
        scan(std::integral_constant<int, 0>{}, std::integral_constant<int, 2>{});
      else
        scan(std::integral_constant<int, 1>{}, std::integral_constant<int, 2>{});
    } else {
      scan(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{});
    }
  } else if (nloc == 0) {
    return;
  } else if (role == SR_OUT) {
    // ================================================================ OUT
    // o is formed transposed: o^T = u^T P^T + (Q S)^T diag(e^b).  The
    // operand fragments are the same registers as for P u and Q S with A
    // and B exchanged (an A fragment holds row lane % 16 over contraction
    // slots, a B fragment column lane % 16 over the same slots), and the
    // accumulator then holds 4 consecutive o columns (v) of one row (t) per
    // lane: o goes out with one 4-element store per lane and tile.
    const int c2 = ridx;
    const float one = opaque_one();
    f32x4 oq[2] = {z4, z4};  // (Q S)^T: lane (n, gq) holds v = 4 gq + i of row t = 16 mt + n
    // 16-bit o after the exchange: lane (n, gq) stores columns 8 (gq / 2) ..
    // + 7 of row orow (of each chunk)
    const int orow = n + 16 * (gq & 1);
    const int64_t o_eb = p.o_dtype == GDN_DTYPE_F32 ? 4 : 2;
    const int64_t o_row_bytes = p.so[1] * o_eb;
    char* const o_lane = static_cast<char*>(p.o) +
                         (head_base(rs, hi, p.so) + (int64_t)orow * p.so[1] + v0 + 16 * c2 + 8 * (gq >> 1)) * o_eb;
    PS_DECL;
    // Operands of o for chunk it (u, P, e^b), read at the start of
    // iteration it + 1 before anything waits on them.
    struct OutOps {
      f32x4 u0, u1;
      f16x8 pAs[2], pLs[2];
      float ebt[2];
      float rat, osc;  // bf16: Q S's factor and o's scale (with the shift)
    };
    auto load_o = [&](int it, OutOps& o) __attribute__((always_inline)) {
      o.u0 = s.uo[it & 1][c2][0][lane];
      o.u1 = s.uo[it & 1][c2][1][lane];  // split SCAN: u as fp16 hi, residual
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        o.pAs[mt] = s.p[it & 1][mt][lane];
        o.pLs[mt] = s.plo[it & 1][mt][lane];
      }
      const float* ebr = reinterpret_cast<const float*>(s.rec[it % RR] + R_EB);
      o.ebt[0] = ebr[n];
      o.ebt[1] = ebr[16 + n];
      if constexpr (BF) {
        o.rat = s.usc[it & 1][c2][0];
        o.osc = s.usc[it & 1][c2][1];
      }
    };
    auto store_chunk = [&](int it, const OutOps& o) __attribute__((always_inline)) {
      f16x8 uh, ul;
      if constexpr (SPLIT) {
        uh = __builtin_bit_cast(f16x8, o.u0);
        ul = __builtin_bit_cast(f16x8, o.u1);
      } else {
        uh = M::from_acc(o.u0, o.u1);
        ul = split_lo_mix(o.u0, o.u1, uh, one);
      }
      f32x4 ov[2];
      PS_BEGIN(uh, ul);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        f32x4 pu = M::mma(ul, o.pAs[mt], z4);
        pu = M::mma(uh, o.pLs[mt], pu);
        pu = M::mma(uh, o.pAs[mt], pu);
        if constexpr (BF)
          ov[mt] = (pu + (o.ebt[mt] * o.rat) * oq[mt]) * o.osc;
        else
          ov[mt] = (pu + o.ebt[mt] * oq[mt]) * p.scale;
      }
      PS_END_B(ov[0], ov[1]);
      const int t0 = (p.c0 + it) * C;
      if (p.o_vec && p.o_dtype != GDN_DTYPE_F32) {
        // 16-bit o: the lanes of 16-lane groups gq and gq ^ 1 exchange a
        // tile (v_permlane16_swap), so that each lane holds 8 consecutive
        // columns of one row: row n of tile 0 in even groups, of tile 1 in
        // odd groups.  One 16-byte store per lane.
        uint32_t w0[2], w1[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (p.o_dtype == GDN_DTYPE_F16) {
            w0[h] = pack_f16x2(ov[0][2 * h], ov[0][2 * h + 1]);
            w1[h] = pack_f16x2(ov[1][2 * h], ov[1][2 * h + 1]);
          } else {
            w0[h] = (uint32_t)float_to_bf16_bits(ov[0][2 * h]) | ((uint32_t)float_to_bf16_bits(ov[0][2 * h + 1]) << 16);
            w1[h] = (uint32_t)float_to_bf16_bits(ov[1][2 * h]) | ((uint32_t)float_to_bf16_bits(ov[1][2 * h + 1]) << 16);
          }
          const auto sw = __builtin_amdgcn_permlane16_swap(w0[h], w1[h], false, false);
          w0[h] = sw[0];
          w1[h] = sw[1];
        }
        if (t0 + orow < T)
          *reinterpret_cast<uint4*>(o_lane + (int64_t)t0 * o_row_bytes) = uint4{w0[0], w0[1], w1[0], w1[1]};
      } else {
        const int64_t o_col = head_base(rs, hi, p.so) + v0 + 16 * c2 + 4 * gq;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const int t = t0 + 16 * mt + n;
          if (t < T) {
            const int64_t off = o_col + (int64_t)t * p.so[1];
            if (p.o_dtype == GDN_DTYPE_F16)
              store_o4<f16>(p.o, off, ov[mt], p.o_vec);
            else if (p.o_dtype == GDN_DTYPE_BF16)
              store_o4<bf16_t>(p.o, off, ov[mt], p.o_vec);
            else
              store_o4<float>(p.o, off, ov[mt], p.o_vec);
          }
        }
      }
    };
    // q rows of chunk it + 1 are read during chunk it (published two ahead)
    auto load_q = [&](int it, f16x8 (&qA)[2][KB]) __attribute__((always_inline)) {
      const int sl = it % R;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) qA[mt][kb] = staged(s.rq[sl], 16 * mt + n, 4 * kb + gq);
    };
    auto chunk = [&](int it, f16x8 (&qA)[2][KB], f16x8 (&qN)[2][KB]) __attribute__((always_inline)) {
      OutOps oo;
      if (it >= 1) load_o(it - 1, oo);
      f16x8 sOp[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) sOp[kb] = s.so[it & 1][c2][kb][lane];
      load_q(min(it + 1, nloc - 1), qN);
      if (it >= 1) store_chunk(it - 1, oo);
      PS_BEGIN(qA[0][0], qA[1][0], sOp[0], sOp[KB - 1]);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        f32x4 acc = z4;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) acc = M::mma(sOp[kb], qA[mt][kb], acc);
        oq[mt] = acc;
      }
      PS_END_A(oq[0], oq[1]);
      wg_barrier();
    };
    f16x8 qa[2][KB], qb[2][KB];
    wg_barrier();
    load_q(0, qa);
    for (int it = 0; it < nloc; it += 2) {
      chunk(it, qa, qb);
      if (it + 1 < nloc) chunk(it + 1, qb, qa);
    }
    {
      OutOps oo;
      load_o(nloc - 1, oo);
      store_chunk(nloc - 1, oo);
    }
    PS_RECORD(2, nloc, 2 * KB, 6);
    PS_RECORD_BAR(2);
  } else if (role == SR_PQK) {
    // ================================================================ PQK
    // Chunk it + 1's q and k rows and gates are read into a second register
    // set while chunk it computes (the LOAD wave publishes chunks two
    // ahead), so no product waits on LDS.
    const float one = opaque_one();
    PS_DECL;
    struct PqkOps {
      f16x8 qf[2][KB], kf[2][KB];
      float bt[2];   // b log2(e) of rows t = 16 mt + n
      f32x4 bj[2];   // of rows j = 16 a + 4 gq + i
    };
    auto read_ops = [&](int it, PqkOps& o) __attribute__((always_inline)) {
      const int sl = it % R;
      const float* bb = reinterpret_cast<const float*>(s.rec[it % RR] + R_B);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          o.qf[mt][kb] = staged(s.rq[sl], 16 * mt + n, 4 * kb + gq);
          o.kf[mt][kb] = staged(s.rk[sl], 16 * mt + n, 4 * kb + gq);
        }
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        o.bt[mt] = bb[16 * mt + n];
        o.bj[mt] = *reinterpret_cast<const f32x4*>(bb + 16 * mt + 4 * gq);
      }
    };
    auto chunk = [&](int it, PqkOps& o, PqkOps& nx) __attribute__((always_inline)) {
      read_ops(min(it + 1, nloc - 1), nx);  // the last chunk's again at the end
      // P^T tiles (rows j, columns t) = K Q^T: the tiles of rows j in
      // [0,16) and [16,32) of one column tile form one P operand
      PS_BEGIN(o.qf[0][0], o.qf[1][0], o.kf[0][0], o.kf[1][0]);
      f16x8 phs[2], pls[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int t = 16 * mt + n;
        f32x4 pt[2] = {z4, z4};
#pragma unroll
        for (int a = 0; a <= mt; ++a) {
          f32x4 acc = z4;
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) acc = M::mma(o.kf[a][kb], o.qf[mt][kb], acc);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            // e^{b_t - b_j} = 2^{(b_t - b_j) log2 e}; the mask folded into
            // the exponent: 2^-inf = 0
            const float x = t >= 16 * a + 4 * gq + i ? o.bt[mt] - o.bj[a][i] : -__builtin_inff();
            pt[a][i] = pin(acc[i] * __builtin_amdgcn_exp2f(x));
          }
        }
        phs[mt] = M::from_acc(pt[0], pt[1]);
        pls[mt] = split_lo_mix(pt[0], pt[1], phs[mt], one);
      }
      PS_END_A(phs[0], phs[1], pls[0], pls[1]);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        s.p[it & 1][mt][lane] = phs[mt];
        s.plo[it & 1][mt][lane] = pls[mt];
      }
      wg_barrier();
    };
    PqkOps oa, ob;
    wg_barrier();
    read_ops(0, oa);
    for (int it = 0; it < nloc; it += 2) {
      chunk(it, oa, ob);
      if (it + 1 < nloc) chunk(it + 1, ob, oa);
    }
    PS_RECORD(3, nloc, 3 * KB, 0);
    PS_RECORD_BAR(3);
  } else {
    // =============================================================== LOAD
    // chunk j -> slots j % R (q, k, v) and j % RR (record).  Rows past the
    // end re-read the last row (finite values that the record's zero beta
    // and the masks cancel).
    constexpr int RCH = K / 8;               // 16-byte pieces per q / k row
    constexpr int NQ = C * RCH / 64;         // DMA copies per q / k tile
    constexpr int VCH = BV / 8;              // pieces per v row
    constexpr int NV = C * VCH / 64;         // DMA copies per v tile
    auto issue = [&](int it) {
      const int j = p.c0 + it;
      const int row0 = j * C;
      const int last = T - 1 - row0;          // rows > last re-read row last
      const char* vb = vh + (int64_t)row0 * svb;
      const int sl = it % R;
      if constexpr (std::is_same<TIn, bf16_t>::value) {
        // k from the record's fp16 copy (rows past the end already repeat
        // the last row)
        const char* const kb = rech + (int64_t)it * RS + R_K16;
        const char* qb = qh + (int64_t)row0 * sqb;
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
          const int pc = 64 * i + lane, r = pc / RCH, cc = swz<K>(r, pc % RCH);  // swz is an involution
          const uint32_t rr = (uint32_t)min(r, last);
          dma16(qb + rr * sqb + cc * 16, &s.rq[sl][0][0] + 64 * i);
          dma16(kb + 16 * frag_piece<K>(r, cc), &s.rk[sl][0][0] + 64 * i);
        }
      } else {
        const char* qb = qh + (int64_t)row0 * sqb;
        const char* kb = kh + (int64_t)row0 * skb;
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
          const int pc = 64 * i + lane, r = pc / RCH, cc = swz<K>(r, pc % RCH);  // swz is an involution
          const uint32_t rr = (uint32_t)min(r, last);
          dma16(qb + rr * sqb + cc * 16, &s.rq[sl][0][0] + 64 * i);
          dma16(kb + rr * skb + cc * 16, &s.rk[sl][0][0] + 64 * i);
        }
      }
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int pc = 64 * i + lane, r = pc / VCH, cc = pc % VCH;
        const uint32_t rr = (uint32_t)min(r, last);
        dma16(vb + rr * svb + cc * 16, &s.rv[sl][0][0] + 64 * i);
      }
      const char* rsrc = rech + (int64_t)it * RS;
#pragma unroll
      for (int i = 0; i < REC_BYTES / 1024; ++i) dma16(rsrc + 1024 * i + 16 * lane, s.rec[it % RR] + 1024 * i);
    };
    // Chunks 0 and 1 are published at the first barrier, and chunk it + 2
    // at iteration it's: the SCAN wave reads chunk it + 1's operands during
    // iteration it.
    // bf16 inputs: once chunk it's copies have landed, its q tile is
    // converted to fp16 in place, before the barrier that publishes it (k
    // arrives in fp16 from the record; the SCAN waves read v's bf16 bits).
    auto convert = [&](int it) __attribute__((always_inline)) {
      if constexpr (BF) {
        if (it >= nloc) return;
        constexpr int NPQ = C * K / 8 / 64;
        f16x8* const q8 = &s.rq[it % R][0][0];
        f16x8 xq[NPQ];
#pragma unroll
        for (int i = 0; i < NPQ; ++i) xq[i] = q8[64 * i + lane];
#pragma unroll
        for (int i = 0; i < NPQ; ++i) q8[64 * i + lane] = to_f16x8<TIn>(__builtin_bit_cast(uint4, xq[i]));
      }
    };
    for (int it = 0; it < D; ++it)
      if (it < nloc) issue(it);
    if (nloc >= D)
      wait_vm<(D - 2) * ND>();
    else
      wait_vm<0>();
    convert(0);
    convert(1);
    wg_barrier();
    for (int it = 0; it < nloc; ++it) {
      if (it + D < nloc) {
        issue(it + D);
        wait_vm<(D - 2) * ND>();
      } else {
        wait_vm<0>();
      }
      convert(it + 2);
      wg_barrier();
    }
    PS_RECORD_BAR(4);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

template <typename TIn, int K, int BV>
int launch_kb(const SArgs& a, int units, hipStream_t s) {
  static_assert(sizeof(ScanSmem<K, BV>) <= kLdsLimit, "LDS budget");
  if (a.nrec > 0) hipLaunchKernelGGL((rec32_kernel<TIn, K>), dim3((a.nrec + 7) / 8), dim3(256), 0, s, a);
  if constexpr (scan_split_ok<TIn, K, BV>()) {
    if (a.L <= kSplitChunks) {
      hipLaunchKernelGGL((scan32_kernel<TIn, K, BV, true>), dim3(units), dim3(64 * scan_waves<BV, true>()), 0, s, a);
      return (int)hipGetLastError();
    }
  }
  hipLaunchKernelGGL((scan32_kernel<TIn, K, BV, false>), dim3(units), dim3(64 * scan_waves<BV, false>()), 0, s, a);
  return (int)hipGetLastError();
}

template <typename TIn>
int launch_t(const SArgs& a, int K, int bv, int units, hipStream_t s) {
  if (K == 64 && bv == 16) return launch_kb<TIn, 64, 16>(a, units, s);
  if (K == 64 && bv == 32) return launch_kb<TIn, 64, 32>(a, units, s);
  if (K == 128 && bv == 16) return launch_kb<TIn, 128, 16>(a, units, s);
  if (K == 128 && bv == 32) return launch_kb<TIn, 128, 32>(a, units, s);
  return GDN_ERR_UNSUPPORTED;
}

}  // namespace s32

bool scan32_supported(int dtype, int K, int C, int BV, int V) {
  return (dtype == GDN_DTYPE_F16 || dtype == GDN_DTYPE_BF16) && C == s32::C && (K == 64 || K == 128) &&
         (BV == 16 || BV == 32);
}

int64_t scan32_record_bytes(int dtype, int K) {
  if (dtype != GDN_DTYPE_BF16) return s32::REC_BYTES;
  return K == 64 ? s32::rec_stride<bf16_t, 64>() : s32::rec_stride<bf16_t, 128>();
}

// Enqueues the segments of one call: for each, the records then the scan
// (arguments checked by the caller; seg_chunks >= 1).
int scan32_launch(const GdnFwdParams& P, int bv, int seg_chunks, hipStream_t stream) {
  s32::SArgs a = {};
  a.q = P.q; a.k = P.k; a.v = P.v; a.g = P.g; a.beta = P.beta; a.h0 = P.h0;
  a.o = P.o; a.fs = P.final_state;
  a.rec = static_cast<char*>(P.workspace);
  for (int d = 0; d < 3; ++d) {
    a.sq[d] = P.q_stride[d]; a.sk[d] = P.k_stride[d]; a.sv[d] = P.v_stride[d];
    a.sg[d] = P.g_stride[d]; a.sb[d] = P.beta_stride[d]; a.so[d] = P.o_stride[d];
  }
  for (int d = 0; d < 4; ++d) { a.sh0[d] = P.h0_stride[d]; a.sfs[d] = P.fs_stride[d]; }
  a.B = P.B; a.T = P.T; a.H = P.H; a.V = P.V; a.nv = P.V / bv;
  a.scale = P.scale;
  a.g_dtype = P.g_dtype; a.beta_dtype = P.beta_dtype; a.o_dtype = P.o_dtype;
  a.cu = P.cu_seqlens;
  const int64_t units = (int64_t)P.B * P.H * a.nv;
  a.xcd_remap = (units % 8 == 0) ? 1 : 0;
  {
    // 16-byte stores of o: 8 consecutive 16-bit elements or 4 fp32 ones
    // per lane (base 16-byte aligned, every stride a multiple of that many
    // elements)
    const int64_t per = P.o_dtype == GDN_DTYPE_F32 ? 4 : 8;
    a.o_vec = reinterpret_cast<uintptr_t>(P.o) % 16 == 0 && P.o_stride[0] % per == 0 &&
              P.o_stride[1] % per == 0 && P.o_stride[2] % per == 0;
  }
  // every sequence has at most ceil(T / C) chunks (the offsets are not read here)
  const int nchmax = (P.T + s32::C - 1) / s32::C;
  const int L = nchmax > 0 ? (seg_chunks < nchmax ? seg_chunks : nchmax) : 1;
  const int nseg = nchmax > 0 ? (nchmax + L - 1) / L : 1;
  a.L = L;
  a.nrec = (int)((int64_t)P.B * P.H * L);
  for (int sg = 0; sg < nseg; ++sg) {
    a.c0 = sg * L;
    a.first = sg == 0;
    if (nchmax == 0) a.nrec = 0;
    int st;
    if (P.qkv_dtype == GDN_DTYPE_F16)
      st = s32::launch_t<f16>(a, P.K, bv, (int)units, stream);
    else if (P.qkv_dtype == GDN_DTYPE_BF16)
      st = s32::launch_t<bf16_t>(a, P.K, bv, (int)units, stream);
    else
      st = GDN_ERR_UNSUPPORTED;
    if (st != 0) return st;
  }
  return GDN_OK;
}

}  // namespace gdn

#ifdef GDN_PHASE_STAMPS
// ---------------------------------------------------------------------------
// MFMA rate probe of the stamps build: every wave issues `n` groups of four
// v_mfma_f32_16x16x32_f16 on independent accumulators between two stamps,
// so (stamped cycles) / (4 n) is the cycles one MFMA keeps a SIMD busy.
// ---------------------------------------------------------------------------
namespace gdn {
__global__ __launch_bounds__(256) void phase_mfma_probe_kernel(float* out, unsigned long long* cyc, int n) {
  using M = Mma<f16>;
  const int lane = threadIdx.x & 63;
  f16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (f16)(0.001f * (lane + i));
    b[i] = (f16)(0.002f * (i - lane));
  }
  f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = c0, c2 = c0, c3 = c0;
  const unsigned long long t0 = s32::ps_stamp(a, b);
  for (int i = 0; i < n; ++i) {
    c0 = M::mma(a, b, c0);
    c1 = M::mma(a, b, c1);
    c2 = M::mma(a, b, c2);
    c3 = M::mma(a, b, c3);
  }
  const unsigned long long t1 = s32::ps_stamp(c0, c1, c2, c3);
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  out[w * 64 + lane] = c0[0] + c1[1] + c2[2] + c3[3];
  if (lane == 0) cyc[w] = t1 - t0;
}
}  // namespace gdn

extern "C" int gdn_phase_mfma_probe(float* out, unsigned long long* cyc, int blocks, int n, void* stream) {
  hipLaunchKernelGGL(gdn::phase_mfma_probe_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, out, cyc, n);
  return (int)hipGetLastError();
}

// Copies the stamp sums of the last call out: scan [1024][8][8], records [16384][4].
extern "C" int gdn_phase_read(void* scan, void* rec) {
  hipError_t e = hipMemcpyFromSymbol(scan, HIP_SYMBOL(gdn::s32::g_phase_scan), sizeof(gdn::s32::g_phase_scan), 0,
                                     hipMemcpyDeviceToHost);
  if (e != hipSuccess) return (int)e;
  return (int)hipMemcpyFromSymbol(rec, HIP_SYMBOL(gdn::s32::g_phase_rec), sizeof(gdn::s32::g_phase_rec), 0,
                                  hipMemcpyDeviceToHost);
}

// Clears the stamp sums (so that waves of an earlier, larger call do not remain).
extern "C" int gdn_phase_clear(void) {
  static unsigned long long zs[gdn::s32::PS_WG * gdn::s32::PS_WAVES * gdn::s32::PS_SLOTS];
  static unsigned long long zr[gdn::s32::PS_REC * 4];
  hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(gdn::s32::g_phase_scan), zs, sizeof(zs), 0, hipMemcpyHostToDevice);
  if (e != hipSuccess) return (int)e;
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(gdn::s32::g_phase_rec), zr, sizeof(zr), 0, hipMemcpyHostToDevice);
}
#endif
