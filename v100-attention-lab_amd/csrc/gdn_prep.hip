// Fused input preparation for the GDN forward (the step before the path):
//   q, k rows  x / sqrt(sum x^2 + eps), the sum of squares in fp32 and the
//              denominator rounded to x's dtype before the division
//              (gdn_ref.py:24-25);
//   beta       sigmoid(x);
//   g          logsigmoid(x)  (the gate recipe of the benchmark inputs).
// One launch reads every input once and writes every output once: HBM-bound
// elementwise work with a 16-lane (K = 128, 16-bit) row reduction.

#include "gdn_fwd_kernel.h"

namespace gdn {
namespace prep {

constexpr int kPrepThreads = 256;
constexpr int kRowUnroll = 4;     // row groups per lane in flight
constexpr int kMaxRowWg = 1024;   // workgroups per row tensor (grid stride beyond)

struct PArgs {
  // row tensors ([B,T,H,K]), compacted: the first nx of {q, k} given
  const void* xin[2];
  void* xout[2];
  int64_t sin[2][3], sout[2][3];
  // gate tensors ([B,T,H]): 0 = beta (sigmoid), 1 = g (logsigmoid)
  const void* gin[2];
  void* gout[2];
  int64_t gsin[2][3], gsout[2][3];
  int gdt_in[2], gdt_out[2];
  uint32_t B, T, H, R;  // R = B T H < 2^31
  float eps;
  int nx;               // row tensors given (0..2)
  int nbr;              // workgroups per row tensor
  int nbg;              // workgroups on the gates
};

template <typename TIn>
struct Lanes;
template <>
struct Lanes<f16> {
  static constexpr int E = 8;
  __device__ static void unpack(const uint4& r, float* x) {
    const f16x8 h = __builtin_bit_cast(f16x8, r);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (float)h[e];
  }
  __device__ static uint4 pack(const float* y) {
    f16x8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (f16)y[e];
    return __builtin_bit_cast(uint4, h);
  }
  __device__ static float round(float d) { return (float)(f16)d; }
};
template <>
struct Lanes<bf16_t> {
  static constexpr int E = 8;
  __device__ static void unpack(const uint4& r, float* x) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = __uint_as_float(w[e] << 16);
      x[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
    }
  }
  __device__ static uint4 pack(const float* y) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = (uint32_t)float_to_bf16_bits(y[2 * e]) | ((uint32_t)float_to_bf16_bits(y[2 * e + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
  __device__ static float round(float d) { return bf16_bits_to_float(float_to_bf16_bits(d)); }
};
template <>
struct Lanes<float> {
  static constexpr int E = 4;
  __device__ static void unpack(const uint4& r, float* x) {
    x[0] = __uint_as_float(r.x);
    x[1] = __uint_as_float(r.y);
    x[2] = __uint_as_float(r.z);
    x[3] = __uint_as_float(r.w);
  }
  __device__ static uint4 pack(const float* y) {
    return make_uint4(__float_as_uint(y[0]), __float_as_uint(y[1]), __float_as_uint(y[2]),
                      __float_as_uint(y[3]));
  }
  __device__ static float round(float d) { return d; }
};

// Element offset of row r = (b T + t) H + h under (b, t, h) strides s.
__device__ __forceinline__ int64_t row_offset(uint32_t r, uint32_t T, uint32_t H, const int64_t* s) {
  const uint32_t bt = r / H, h = r - bt * H;
  const uint32_t b = bt / T, t = bt - b * T;
  return (int64_t)b * s[0] + (int64_t)t * s[1] + (int64_t)h * s[2];
}

// L lanes hold one row (16 bytes each); a wave covers 64 / L rows per group
// and kRowUnroll groups per pass, consecutive rows.
template <typename TIn, int K>
__device__ void norm_rows(const PArgs& p, int x, uint32_t blk) {
  using Lx = Lanes<TIn>;
  constexpr int E = Lx::E, L = K / E, RPW = 64 / L, U = kRowUnroll;
  static_assert(L >= 1 && L <= 64 && 64 % L == 0, "row width");
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int sub = lane / L, pc = lane % L;
  const char* xin = static_cast<const char*>(p.xin[x]);
  char* xout = static_cast<char*>(p.xout[x]);
  const uint32_t step = (uint32_t)p.nbr * (kPrepThreads / 64) * RPW * U;
  for (uint32_t r0 = (blk * (kPrepThreads / 64) + wv) * RPW * U; r0 < p.R; r0 += step) {
    uint4 raw[U];
    int64_t oo[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t r = r0 + u * RPW + sub;
      raw[u] = make_uint4(0u, 0u, 0u, 0u);
      oo[u] = 0;
      ok[u] = r < p.R;
      if (ok[u]) {
        const int64_t io = (row_offset(r, p.T, p.H, p.sin[x]) + pc * E) * (int64_t)sizeof(TIn);
        oo[u] = (row_offset(r, p.T, p.H, p.sout[x]) + pc * E) * (int64_t)sizeof(TIn);
        raw[u] = *reinterpret_cast<const uint4*>(xin + io);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float v[E];
      Lx::unpack(raw[u], v);
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) ss = __builtin_fmaf(v[e], v[e], ss);
#pragma unroll
      for (int o = L / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
      const float d = Lx::round(sqrtf(ss + p.eps));
#pragma unroll
      for (int e = 0; e < E; ++e) v[e] = v[e] / d;
      if (ok[u]) *reinterpret_cast<uint4*>(xout + oo[u]) = Lx::pack(v);
    }
  }
}

__device__ __forceinline__ float sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

// log(sigmoid(x)) = min(x, 0) - log(1 + e^{-|x|}), finite for every x.
__device__ __forceinline__ float logsigmoid(float x) {
  return fminf(x, 0.f) - log1pf(expf(-fabsf(x)));
}

__device__ void gates(const PArgs& p, uint32_t blk) {
  const uint32_t step = (uint32_t)p.nbg * kPrepThreads;
  for (uint32_t r = blk * kPrepThreads + threadIdx.x; r < p.R; r += step) {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      if (p.gin[w] == nullptr) continue;
      const float xv = load_scalar(p.gin[w], row_offset(r, p.T, p.H, p.gsin[w]), p.gdt_in[w]);
      const float y = w == 0 ? sigmoid(xv) : logsigmoid(xv);
      store_scalar(p.gout[w], row_offset(r, p.T, p.H, p.gsout[w]), p.gdt_out[w], y);
    }
  }
}

template <typename TIn, int K>
__global__ __launch_bounds__(kPrepThreads) void prep_kernel(const PArgs p) {
  const uint32_t b = blockIdx.x;
  const uint32_t nrow = (uint32_t)p.nx * p.nbr;
  if (b < nrow)
    norm_rows<TIn, K>(p, (int)(b / p.nbr), b % p.nbr);
  else
    gates(p, b - nrow);
}

template <typename TIn>
int launch_t(const PArgs& a, int K, int grid, hipStream_t s) {
  switch (K) {
    case 32: hipLaunchKernelGGL((prep_kernel<TIn, 32>), dim3(grid), dim3(kPrepThreads), 0, s, a); break;
    case 64: hipLaunchKernelGGL((prep_kernel<TIn, 64>), dim3(grid), dim3(kPrepThreads), 0, s, a); break;
    case 128: hipLaunchKernelGGL((prep_kernel<TIn, 128>), dim3(grid), dim3(kPrepThreads), 0, s, a); break;
    case 256: hipLaunchKernelGGL((prep_kernel<TIn, 256>), dim3(grid), dim3(kPrepThreads), 0, s, a); break;
    default: return GDN_ERR_UNSUPPORTED;
  }
  return (int)hipGetLastError();
}

}  // namespace prep
}  // namespace gdn

using namespace gdn;
using namespace gdn::prep;

extern "C" int gdn_prep_launch(const GdnPrepParams* prm, void* stream) {
  if (prm == nullptr) return GDN_ERR_NULL_POINTER;
  const GdnPrepParams& P = *prm;
  if (P.B < 0 || P.T < 0 || P.H < 0) return GDN_ERR_BAD_SHAPE;
  const int64_t R = (int64_t)P.B * P.T * P.H;
  if (R >= 0x7fffffffLL) return GDN_ERR_BAD_SHAPE;
  const bool has_q = P.q_in != nullptr, has_k = P.k_in != nullptr;
  if ((has_q && P.q_out == nullptr) || (has_k && P.k_out == nullptr) ||
      (P.beta_in != nullptr && P.beta_out == nullptr) || (P.g_in != nullptr && P.g_out == nullptr))
    return GDN_ERR_NULL_POINTER;
  if (!valid_dtype(P.beta_in_dtype) || !valid_dtype(P.beta_out_dtype) ||
      !valid_dtype(P.g_in_dtype) || !valid_dtype(P.g_out_dtype))
    return GDN_ERR_BAD_DTYPE;
  if (has_q || has_k) {
    if (!valid_dtype(P.qk_dtype)) return GDN_ERR_BAD_DTYPE;
    if (P.K != 32 && P.K != 64 && P.K != 128 && P.K != 256) return GDN_ERR_UNSUPPORTED;
    const int eb = elem_bytes(P.qk_dtype);
    const void* ptrs[4] = {P.q_in, P.q_out, P.k_in, P.k_out};
    const int64_t* strides[4] = {P.q_in_stride, P.q_out_stride, P.k_in_stride, P.k_out_stride};
    for (int i = 0; i < 4; ++i) {
      if (ptrs[i] == nullptr) continue;
      if (reinterpret_cast<uintptr_t>(ptrs[i]) % 16 != 0) return GDN_ERR_MISALIGNED;
      for (int d = 0; d < 3; ++d)
        if ((strides[i][d] * eb) % 16 != 0) return GDN_ERR_MISALIGNED;
    }
  }
  if (R == 0) return GDN_OK;

  PArgs a = {};
  a.B = P.B; a.T = P.T; a.H = P.H; a.R = (uint32_t)R;
  a.eps = P.eps;
  int nx = 0;
  auto add_rows = [&](const void* in, void* out, const int64_t* si, const int64_t* so) {
    a.xin[nx] = in;
    a.xout[nx] = out;
    for (int d = 0; d < 3; ++d) { a.sin[nx][d] = si[d]; a.sout[nx][d] = so[d]; }
    ++nx;
  };
  if (has_q) add_rows(P.q_in, P.q_out, P.q_in_stride, P.q_out_stride);
  if (has_k) add_rows(P.k_in, P.k_out, P.k_in_stride, P.k_out_stride);
  a.nx = nx;
  const void* gin[2] = {P.beta_in, P.g_in};
  void* gout[2] = {P.beta_out, P.g_out};
  const int64_t* gsi[2] = {P.beta_in_stride, P.g_in_stride};
  const int64_t* gso[2] = {P.beta_out_stride, P.g_out_stride};
  const int gdi[2] = {P.beta_in_dtype, P.g_in_dtype}, gdo[2] = {P.beta_out_dtype, P.g_out_dtype};
  bool any_gate = false;
  for (int w = 0; w < 2; ++w) {
    a.gin[w] = gin[w];
    a.gout[w] = gout[w];
    a.gdt_in[w] = gdi[w];
    a.gdt_out[w] = gdo[w];
    for (int d = 0; d < 3; ++d) { a.gsin[w][d] = gsi[w][d]; a.gsout[w][d] = gso[w][d]; }
    any_gate |= gin[w] != nullptr;
  }
  // Row work: rows per workgroup pass = 4 waves x (64 / lanes per row) x
  // unroll; enough workgroups for several per CU, the rest by grid stride.
  const int K = (nx > 0) ? P.K : 128;
  const int lanes = K * (nx > 0 ? elem_bytes(P.qk_dtype) : 2) / 16;
  const int64_t rows_per_pass = (int64_t)(kPrepThreads / 64) * (64 / lanes) * kRowUnroll;
  a.nbr = nx > 0 ? (int)std::min<int64_t>((R + rows_per_pass - 1) / rows_per_pass, kMaxRowWg) : 0;
  a.nbg = any_gate ? (int)std::min<int64_t>((R + kPrepThreads - 1) / kPrepThreads, 512) : 0;
  const int grid = nx * a.nbr + a.nbg;
  if (grid == 0) return GDN_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int dt = nx > 0 ? P.qk_dtype : GDN_DTYPE_F16;
  switch (dt) {
    case GDN_DTYPE_F16: return launch_t<f16>(a, K, grid, s);
    case GDN_DTYPE_BF16: return launch_t<bf16_t>(a, K, grid, s);
    default: return launch_t<float>(a, K, grid, s);
  }
}
