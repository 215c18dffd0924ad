// Host side of the C ABI declared in include/gdn_mi355x.h: argument checks,
// BV choice and dispatch to the per-dtype launchers.

#include <mutex>

#include "gdn_fwd_kernel.h"

namespace gdn {

// BV choice.  32-row chunks: 32 columns per workgroup when that still
// gives one workgroup per CU (256 CUs), else 16 (fp16 and bf16 alike,
// bench.py --sweep).  Phased kernel: the largest slice that still gives one
// workgroup per CU, else the smallest supported.
int auto_block_v(int B, int H, int K, int V, int C, int dtype) {
  const long long bh = (long long)B * H;
  if (pipe_supported(dtype, K, C, 16) && V % 16 == 0) {
    if (V % 32 == 0 && bh * (V / 32) >= 256) return 32;
    return 16;
  }
  int best = -1;
  for (int bv : {64, 32, 16}) {
    if (V % bv != 0 || !supported(dtype, K, C, bv)) continue;
    if (best < 0) best = bv;
    if (bh * (V / bv) >= 256) return bv;
    best = bv;
  }
  return best;
}

// The pipelined kernel addresses the rows of one chunk as a chunk base plus
// a 32-bit per-lane offset: C rows of q, k, v, g and beta must span less
// than 2^31 bytes (and the row strides must not be negative).
static bool pipe_offsets_fit(const GdnFwdParams& P) {
  const int64_t eb = elem_bytes(P.qkv_dtype);
  const int64_t rows = 32;
  const int64_t lim = 0x7fffffffLL;
  const int64_t row_strides[5] = {P.q_stride[1] * eb, P.k_stride[1] * eb, P.v_stride[1] * eb,
                                  P.g_stride[1] * elem_bytes(P.g_dtype),
                                  P.beta_stride[1] * elem_bytes(P.beta_dtype)};
  for (int64_t s : row_strides)
    if (s < 0 || rows * s + (int64_t)P.K * eb + (int64_t)P.V * eb > lim) return false;
  return true;
}

// The two-launch path for 64-row chunks, unless the phased kernel is asked for.
static bool uses_c64(const GdnFwdParams& P) {
  return !(P.flags & GDN_FLAG_PHASED_KERNEL) && c64_supported(P.K, P.chunk_size, P.V);
}

// Records of at most this many chunks per sequence are what
// gdn_fwd_workspace_size asks for on the 32-row two-launch path.
constexpr int64_t kSegChunks = 256;

// The 32-row two-launch path (records, then the scan) for this BV, unless
// another kernel is asked for.
static bool uses_scan32(const GdnFwdParams& P, int bv) {
  return !(P.flags & (GDN_FLAG_PHASED_KERNEL | GDN_FLAG_FUSED_KERNEL)) &&
         scan32_supported(P.qkv_dtype, P.K, P.chunk_size, bv, P.V) && pipe_offsets_fit(P);
}

// ---------------------------------------------------------------------------
// Static scratch of gdn_fwd_launch_noalloc: the record workspace for callers
// that cannot allocate.  Each device holds its own copy from module load to
// process end; host code uses only the per-device address fetched with
// hipGetSymbolAddress (the array's name is a host-side stand-in).  Every
// call on a device shares that device's copy, so calls that overlap on one
// device race.  The records a call reads are written by the same call first,
// so nothing needs clearing between calls.
constexpr int64_t kScratchBytes = 32ll << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

// Device address of the current device's scratch copy (fetched once per
// device, with that device current).
static int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return GDN_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (ptr == nullptr || reinterpret_cast<uintptr_t>(ptr) % 256 != 0) return GDN_ERR_WORKSPACE;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace gdn

using namespace gdn;

// The launch of gdn_fwd_launch and gdn_fwd_launch_noalloc.  With
// `scratch_bytes` > 0 the record workspace is the library's static scratch
// array (its device address fetched only after every argument check passed)
// and params->workspace is ignored.
static int launch_impl(const GdnFwdParams& P, hipStream_t s, int64_t scratch_bytes) {
  if (P.B <= 0 || P.H <= 0 || P.K <= 0 || P.V <= 0 || P.T < 0 || P.V % 16 != 0)
    return GDN_ERR_BAD_SHAPE;
  if (!valid_dtype(P.qkv_dtype) || !valid_dtype(P.g_dtype) || !valid_dtype(P.beta_dtype) ||
      !valid_dtype(P.o_dtype))
    return GDN_ERR_BAD_DTYPE;
  if (P.final_state == nullptr) return GDN_ERR_NULL_POINTER;
  if (P.T > 0 && (P.q == nullptr || P.k == nullptr || P.v == nullptr || P.g == nullptr ||
                  P.beta == nullptr || P.o == nullptr))
    return GDN_ERR_NULL_POINTER;
  bool c64 = uses_c64(P);
  int bv = c64 ? 16 : P.block_v;
  if (bv == 0) bv = auto_block_v(P.B, P.H, P.K, P.V, P.chunk_size, P.qkv_dtype);
  if (!c64 && (bv <= 0 || P.V % bv != 0 || !supported(P.qkv_dtype, P.K, P.chunk_size, bv)))
    return GDN_ERR_UNSUPPORTED;
  // 16-byte rows for the vector loads of q, k, v.
  const int eb = elem_bytes(P.qkv_dtype);
  const void* ptrs[3] = {P.q, P.k, P.v};
  const int64_t* strides[3] = {P.q_stride, P.k_stride, P.v_stride};
  if (P.T > 0) {
    for (int i = 0; i < 3; ++i) {
      if (reinterpret_cast<uintptr_t>(ptrs[i]) % 16 != 0) return GDN_ERR_MISALIGNED;
      for (int d = 0; d < 3; ++d)
        if ((strides[i][d] * eb) % 16 != 0) return GDN_ERR_MISALIGNED;
    }
  }
  const long long units = (long long)P.B * P.H * (P.V / bv);
  if (units > 0x7fffffffLL) return GDN_ERR_BAD_SHAPE;
  bool scan32 = uses_scan32(P, bv) && (scratch_bytes > 0 || P.workspace != nullptr);
  if (scratch_bytes > 0 && P.T > 0) {
    // The static scratch must hold one chunk's records per sequence and
    // head (longer sequences run in segments).  Where it cannot, the call
    // runs on a kernel that needs no workspace: the fused kernel for
    // 32-row chunks (it supports every shape the records path does), the
    // phased kernel for 64-row chunks.
    const int64_t bh = (int64_t)P.B * P.H;
    if (scan32 && bh * scan32_record_bytes(P.qkv_dtype, P.K) > scratch_bytes) scan32 = false;
    if (c64 && bh * c64_record_bytes(P.K, P.qkv_dtype) > scratch_bytes) {
      if (!supported(P.qkv_dtype, P.K, P.chunk_size, bv)) return GDN_ERR_SCRATCH_LIMIT;
      c64 = false;
    }
  }
  // workspace: the caller's, or the static scratch array
  GdnFwdParams W = P;
  if (scratch_bytes > 0 && (c64 || scan32) && P.T > 0) {
    void* ptr = nullptr;
    const int st = scratch_address(&ptr);
    if (st != 0) return st;
    W.workspace = ptr;
    W.workspace_bytes = scratch_bytes;
  }
  // Launch errors are read back with hipGetLastError after each launch:
  // clear one left by unrelated earlier work so that it is not reported
  // as this call's.
  (void)hipGetLastError();
  if (c64) {
    // segment length: as many chunks per sequence as the workspace holds
    const int64_t per_chunk = (int64_t)P.B * P.H * c64_record_bytes(P.K, P.qkv_dtype);
    const int64_t L = W.workspace == nullptr ? 0 : W.workspace_bytes / per_chunk;
    if (P.T > 0 && (reinterpret_cast<uintptr_t>(W.workspace) % 256 != 0 || L < 1)) return GDN_ERR_WORKSPACE;
    return c64_launch(W, (int)(L < 1 ? 1 : L < 0x7fffffff ? L : 0x7fffffff), s);
  }
  if (scan32) {
    // segment length: as many chunks per sequence as the workspace holds
    const int64_t per_chunk = (int64_t)P.B * P.H * scan32_record_bytes(P.qkv_dtype, P.K);
    const int64_t L = W.workspace_bytes / per_chunk;
    if (P.T > 0 && (reinterpret_cast<uintptr_t>(W.workspace) % 256 != 0 || L < 1)) return GDN_ERR_WORKSPACE;
    return scan32_launch(W, bv, (int)(L < 1 ? 1 : L < 0x7fffffff ? L : 0x7fffffff), s);
  }

  KArgs a = {};
  a.q = P.q; a.k = P.k; a.v = P.v; a.g = P.g; a.beta = P.beta; a.h0 = P.h0;
  a.o = P.o; a.fs = P.final_state;
  for (int d = 0; d < 3; ++d) {
    a.sq[d] = P.q_stride[d]; a.sk[d] = P.k_stride[d]; a.sv[d] = P.v_stride[d];
    a.sg[d] = P.g_stride[d]; a.sb[d] = P.beta_stride[d]; a.so[d] = P.o_stride[d];
  }
  for (int d = 0; d < 4; ++d) { a.sh0[d] = P.h0_stride[d]; a.sfs[d] = P.fs_stride[d]; }
  a.B = P.B; a.T = P.T; a.H = P.H; a.V = P.V; a.nv = P.V / bv;
  a.scale = P.scale;
  a.g_dtype = P.g_dtype; a.beta_dtype = P.beta_dtype; a.o_dtype = P.o_dtype;
  a.xcd_remap = (units % 8 == 0) ? 1 : 0;
  a.cu = P.cu_seqlens;

  const int grid = (int)units;
  if (!(P.flags & GDN_FLAG_PHASED_KERNEL) && pipe_supported(P.qkv_dtype, P.K, P.chunk_size, bv) &&
      pipe_offsets_fit(P)) {
    if (P.qkv_dtype == GDN_DTYPE_F16) return launch_pipe_f16(a, P.K, bv, grid, s);
    return launch_pipe_bf16(a, P.K, bv, grid, s);
  }
  switch (P.qkv_dtype) {
    case GDN_DTYPE_F16: return launch_f16(a, P.K, P.chunk_size, bv, grid, s);
    case GDN_DTYPE_BF16: return launch_bf16(a, P.K, P.chunk_size, bv, grid, s);
    case GDN_DTYPE_F32: return launch_f32(a, P.K, P.chunk_size, bv, grid, s);
    default: return GDN_ERR_BAD_DTYPE;
  }
}

extern "C" {

int gdn_fwd_abi_version(void) { return GDN_MI355X_ABI_VERSION; }

int gdn_fwd_auto_block_v(int B, int H, int K, int V, int chunk_size, int qkv_dtype) {
  if (B <= 0 || H <= 0 || K <= 0 || V <= 0 || V % 16 != 0) return -1;
  return auto_block_v(B, H, K, V, chunk_size, qkv_dtype);
}

const char* gdn_fwd_status_string(int status) {
  switch (status) {
    case GDN_OK: return "success";
    case GDN_ERR_NULL_POINTER: return "gdn_fwd: a required pointer is NULL";
    case GDN_ERR_BAD_SHAPE: return "gdn_fwd: invalid shape (B, H, K, V must be > 0, T >= 0, V % 16 == 0)";
    case GDN_ERR_UNSUPPORTED:
      return "gdn_fwd: unsupported configuration (K in {32,64,128,256}, chunk_size in {32,64}, "
             "block_v in {16,32,64} dividing V, within the 160 KB LDS budget)";
    case GDN_ERR_MISALIGNED:
      return "gdn_fwd: q/k/v rows must be 16-byte aligned with a contiguous last dimension";
    case GDN_ERR_BAD_DTYPE: return "gdn_fwd: unknown dtype code";
    case GDN_ERR_WORKSPACE:
      return "gdn: workspace missing, misaligned or smaller than gdn_fwd_workspace_size() / "
             "gdn_bwd_workspace_size()";
    case GDN_ERR_SCRATCH_LIMIT:
      return "gdn_fwd_launch_noalloc: the call needs more workspace than the static scratch array "
             "(gdn_fwd_scratch_bytes()) holds";
    default: return hipGetErrorString((hipError_t)status);
  }
}

int64_t gdn_fwd_workspace_size(const GdnFwdParams* prm) {
  if (prm == nullptr) return -1;
  const GdnFwdParams& P = *prm;
  if (P.B <= 0 || P.H <= 0 || P.K <= 0 || P.V <= 0 || P.T < 0 || P.V % 16 != 0) return -1;
  if (!valid_dtype(P.qkv_dtype)) return -1;
  if (uses_c64(P)) return c64_workspace_size(P.B, P.T, P.H, P.K, P.cu_seqlens ? P.B : 0, P.qkv_dtype);
  const int bv = P.block_v ? P.block_v : auto_block_v(P.B, P.H, P.K, P.V, P.chunk_size, P.qkv_dtype);
  if (bv > 0 && P.V % bv == 0 && uses_scan32(P, bv)) {
    const int64_t nch = (P.T + 31) / 32;
    const int64_t L = nch < kSegChunks ? nch : kSegChunks;
    const int64_t bytes = (int64_t)P.B * P.H * L * scan32_record_bytes(P.qkv_dtype, P.K);
    return (bytes + 255) / 256 * 256;
  }
  return 0;
}

int gdn_fwd_launch(const GdnFwdParams* prm, void* stream) {
  if (prm == nullptr) return GDN_ERR_NULL_POINTER;
  return launch_impl(*prm, static_cast<hipStream_t>(stream), 0);
}

int gdn_fwd_launch_noalloc(const GdnFwdParams* prm, void* stream) {
  if (prm == nullptr) return GDN_ERR_NULL_POINTER;
  return launch_impl(*prm, static_cast<hipStream_t>(stream), kScratchBytes);
}

int64_t gdn_fwd_scratch_bytes(void) { return kScratchBytes; }

}  // extern "C"
