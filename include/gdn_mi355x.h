/*
 * gdn_mi355x.h -- C ABI of the MI355X (gfx950) fused chunked Gated DeltaNet
 * forward.
 *
 * Replaces the reference's GPU boundary for this path:
 *   - the Python launcher  gdn_chunk_fwd(q, k, v, beta, g) -> (o, h_final)
 *     (gdn_triton.py:113-140), and
 *   - the raw kernel launch _gdn_fwd_kernel.fn[grid](Q, K, V, Beta, G, O, Hf,
 *     <b,t,h strides of every tensor>, T, H, DK, DV, C, BV)
 *     (gdn_triton.py:29-41; bench_gdn.py:43-59).
 * The struct below carries exactly what that launch takes (device pointers,
 * per-tensor (b, t, h) strides, T/H/K/V, chunk size C and V-slice BV) plus
 * what the north-star surface adds (h0, scale, dtypes).
 *
 * Semantics (per batch b and head h; the state S is K x V, S = h^T of the
 * reference's V x K state, gdn_ref.py:3-9):
 *     S_t = e^{g_t} S_{t-1} + k_t u_t^T,
 *     u_t = beta_t (v_t - e^{g_t} S_{t-1}^T k_t),
 *     o_t = scale * S_t^T q_t.
 *
 * Contract:
 *   - All pointers are device pointers on the current HIP device.  The call
 *     only enqueues work on `stream`; it never allocates, never synchronises
 *     and keeps no state between calls (re-entrant).
 *   - Inputs are read-only.  `o` and `final_state` are written in full.
 *   - q, k, v: innermost (K / V) dimension contiguous; base pointer and the
 *     b/t/h strides (in elements) must give 16-byte aligned rows.
 *   - g, beta: any strides.  h0 / final_state: any strides (b, h, k, v).
 *   - h0 may be NULL (zero initial state).
 *   - T may be any value >= 0; a trailing partial chunk is masked in-kernel
 *     (equivalent to the reference's zero padding, gdn_ref.py:102-114).
 *   - cu_seqlens (optional, the variable-length form of FLA's
 *     chunk_gated_delta_rule, called at bench_gdn.py:169-172): B sequences
 *     packed along t of one batch.  Sequence i is rows
 *     [cu_seqlens[i], cu_seqlens[i+1]) of batch 0 of every [B,T,H,*] tensor
 *     (their b stride is unused), with its own h0[i] / final_state[i]; T is
 *     the packed length.  The offsets live in device memory and are not read
 *     on the host; each kernel clamps them to [0, T].
 */
#ifndef GDN_MI355X_H
#define GDN_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 5: C = 32 with fp16 / bf16 inputs runs on per-chunk records in the
 * caller's workspace (gdn_fwd_workspace_size is non-zero there, and a
 * workspace smaller than one record per sequence and head is
 * GDN_ERR_WORKSPACE); 64-row records are laid out per sequence segment. */
#define GDN_MI355X_ABI_VERSION 5

/* Element types of the tensors crossing the boundary. */
enum GdnDtype {
  GDN_DTYPE_F32 = 0,
  GDN_DTYPE_F16 = 1,
  GDN_DTYPE_BF16 = 2
};

/* Status codes.  0 is success; values below 1000 are hipError_t values
 * passed through from the HIP runtime; values from 1000 are argument
 * errors detected before launch (nothing is enqueued).  A launch error
 * (a hipError_t) can come after earlier segments of the same call were
 * enqueued, so o and final_state may then be partly written. */
enum GdnStatus {
  GDN_OK = 0,
  GDN_ERR_NULL_POINTER = 1001,
  GDN_ERR_BAD_SHAPE = 1002,
  GDN_ERR_UNSUPPORTED = 1003,
  GDN_ERR_MISALIGNED = 1004,
  GDN_ERR_BAD_DTYPE = 1005,
  GDN_ERR_WORKSPACE = 1006,
  /* gdn_fwd_launch_noalloc: the call needs more workspace than the static
   * scratch array holds (gdn_fwd_scratch_bytes()) */
  GDN_ERR_SCRATCH_LIMIT = 1007
};

/* Launch options (bit flags). */
enum GdnFlags {
  /* Use the phase-by-phase kernel even where the pipelined one applies
   * (testing and comparison). */
  GDN_FLAG_PHASED_KERNEL = 1,
  /* 32-row chunks: use the single fused pipelined kernel (no workspace)
   * even when a workspace is given (testing and comparison). */
  GDN_FLAG_FUSED_KERNEL = 2
};

typedef struct GdnFwdParams {
  /* inputs: q, k [B,T,H,K]; v [B,T,H,V]; g, beta [B,T,H]; h0 [B,H,K,V] */
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  const float* h0;          /* nullable */
  /* outputs: o [B,T,H,V]; final_state [B,H,K,V] fp32 */
  void* o;
  float* final_state;
  /* strides in elements: (b, t, h) for the [B,T,H,*] tensors */
  int64_t q_stride[3];
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t g_stride[3];
  int64_t beta_stride[3];
  int64_t o_stride[3];
  /* strides in elements: (b, h, k, v) for the state tensors */
  int64_t h0_stride[4];
  int64_t fs_stride[4];
  int32_t B, T, H, K, V;
  float scale;              /* o = scale * S^T q (FLA convention) */
  int32_t chunk_size;       /* C: 32 or 64 */
  int32_t block_v;          /* BV: 16, 32 or 64 dividing V; 0 = auto */
  int32_t qkv_dtype;        /* GdnDtype of q, k, v */
  int32_t g_dtype;          /* GdnDtype of g */
  int32_t beta_dtype;       /* GdnDtype of beta */
  int32_t o_dtype;          /* GdnDtype of o */
  int32_t flags;            /* GdnFlags; 0 = default */
  /* nullable: B + 1 int64 row offsets of packed sequences (device memory) */
  const int64_t* cu_seqlens;
  /* device memory of at least gdn_fwd_workspace_size(params) bytes,
   * 256-byte aligned, owned by the caller; nullable when that size is 0 */
  void* workspace;
  int64_t workspace_bytes;
} GdnFwdParams;

/* Enqueue one chunked GDN forward on `stream` (a hipStream_t; NULL = the
 * legacy default stream).  Returns a GdnStatus / hipError_t value.
 * Replaces gdn_chunk_fwd / _gdn_fwd_kernel (gdn_triton.py:29-140).
 *   - C = 32, fp16 or bf16 q/k/v, K in {64, 128}, with a
 *     workspace, and C = 64 with
 *     K in {32, 64, 128} (any dtype; block_v is 16 there): two launches per
 *     segment of the sequence (per-chunk records of the state-independent
 *     work, then the scan over chunks).  The segment length is what the
 *     workspace holds: workspace_bytes / (B * H * record bytes) chunks per
 *     sequence (at least one), so any workspace of at least
 *     gdn_fwd_workspace_size() bytes runs the call; a longer sequence runs
 *     as several segments, its state passing through final_state in fp32.
 *     C = 64 needs params->workspace.
 *   - C = 32 without a workspace (or GDN_FLAG_FUSED_KERNEL), or K = 256 /
 *     GDN_FLAG_PHASED_KERNEL: one fused kernel, no workspace.
 * The state stays on chip in every path: no chunk state is written. */
int gdn_fwd_launch(const GdnFwdParams* params, void* stream);

/* gdn_fwd_launch without a caller workspace and without any allocation.
 * No counterpart in the reference (its Triton launch needs no workspace);
 * it is for callers that cannot allocate device memory: code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * Same arguments, semantics and statuses as gdn_fwd_launch, except that
 * params->workspace / workspace_bytes are ignored: the paths that take a
 * workspace (32-row records, 64-row records) use a static device array of
 * gdn_fwd_scratch_bytes() bytes (32 MiB) held by each device from the
 * library's load to the end of the process.
 *   - 32-row chunks (fp16, bf16): the sequence runs in segments of as many
 *     chunks as the array holds (B * H records per chunk, of 3 KB for fp16
 *     and 3 KB + 2 C K bytes for bf16, which also carry the chunk's k rows
 *     in fp16).  If one chunk per sequence does not fit (fp16:
 *     B * H > 10922; bf16 at K = 128: B * H > 2978), the call runs on the
 *     fused kernel, which needs no workspace.
 *   - 64-row chunks: likewise in segments (records of 33 KB per chunk and
 *     head for 16-bit inputs, 66 KB for fp32 at K = 128).  If one chunk
 *     per sequence does not fit (B * H > 992 for 16-bit inputs), the call
 *     runs on the phased kernel, which needs no workspace;
 *     GDN_ERR_SCRATCH_LIMIT only where that kernel does not support the
 *     shape either.
 *   - The first call on a device fetches the array's device address
 *     (hipGetSymbolAddress) and keeps it: make one call on each device
 *     before capturing a call into a HIP graph.
 * Every call on a device shares that device's array: calls that overlap
 * on one device (on different streams, or from different host threads)
 * race and must be serialised by the caller. */
int gdn_fwd_launch_noalloc(const GdnFwdParams* params, void* stream);

/* Size in bytes of the static scratch array of gdn_fwd_launch_noalloc. */
int64_t gdn_fwd_scratch_bytes(void);

/* Bytes of workspace gdn_fwd_launch needs for these params (0 for the fused
 * kernels; the records of a segment of at most 256 chunks per sequence for
 * 32-row chunks, at most 64 chunks for 64-row chunks; B = the number of
 * sequences when cu_seqlens is set); -1 if the shape is invalid.  No counterpart in the reference, whose Triton
 * launch needs none. */
int64_t gdn_fwd_workspace_size(const GdnFwdParams* params);

/* The block_v the launcher picks when params->block_v == 0 (for logging and
 * tests); -1 if the shape is unsupported.  No counterpart in the reference,
 * whose autotuner picks BV at run time (gdn_triton.py:18-28). */
int gdn_fwd_auto_block_v(int B, int H, int K, int V, int chunk_size,
                         int qkv_dtype);

/* Fused input preparation, the step before the path: one launch that
 * L2-normalises q and k rows and applies the gate activations of the
 * benchmark's input recipe.  Replaces the reference's _l2norm
 * (gdn_ref.py:24-25: x / sqrt(sum x^2 + eps), the sum in fp32, the
 * denominator rounded to x's dtype before the division; called by
 * bench_gdn.py:35-36) and the beta / g activations of the input recipe
 * (beta = sigmoid(x), g = logsigmoid(x)).
 *   - Each input may be NULL (that output is skipped); an output may alias
 *     its input (in-place).
 *   - q/k in and out: [B,T,H,K], qk_dtype, innermost dim contiguous, 16-byte
 *     aligned rows; K in {32, 64, 128, 256}.
 *   - gates: [B,T,H], any strides, each with its own in / out dtype.
 *   - B * T * H < 2^31.  Same launch contract as gdn_fwd_launch. */
typedef struct GdnPrepParams {
  const void* q_in;
  void* q_out;
  const void* k_in;
  void* k_out;
  const void* beta_in;      /* beta_out = sigmoid(beta_in) */
  void* beta_out;
  const void* g_in;         /* g_out = logsigmoid(g_in) */
  void* g_out;
  /* strides in elements, (b, t, h) */
  int64_t q_in_stride[3];
  int64_t q_out_stride[3];
  int64_t k_in_stride[3];
  int64_t k_out_stride[3];
  int64_t beta_in_stride[3];
  int64_t beta_out_stride[3];
  int64_t g_in_stride[3];
  int64_t g_out_stride[3];
  int32_t B, T, H, K;
  int32_t qk_dtype;         /* GdnDtype of q, k (in and out) */
  int32_t beta_in_dtype;
  int32_t beta_out_dtype;
  int32_t g_in_dtype;
  int32_t g_out_dtype;
  float eps;                /* 1e-6 in the reference */
} GdnPrepParams;

/* Enqueue the input preparation on `stream`; returns a GdnStatus /
 * hipError_t value. */
int gdn_prep_launch(const GdnPrepParams* params, void* stream);

/* Backward of the forward above: gradients of q, k, v, g, beta and h0 given
 * d_o (the gradient of o) and d_final_state.  No counterpart in the
 * reference, whose README lists the backward as future work
 * (README.md:259); it is the gradient of the recurrence gdn_ref.py:3-9 and
 * is checked against reverse-mode differentiation of that recurrence.
 *   - Same tensors, strides and varlen convention as GdnFwdParams; the
 *     chunk length is 32.  K in {32, 64, 128}; V a multiple of 16.
 *   - q, k, v: 16-byte aligned rows as for the forward.  dq, dk, dv (q's
 *     dtype), dg, dbeta (g's / beta's dtypes): any strides.  dh0 [B,H,K,V]
 *     fp32 (nullable: not written).
 *   - d_final_state nullable (zero).  h0 nullable (zero).
 *   - workspace: device memory of at least gdn_bwd_workspace_size_params()
 *     bytes (gdn_bwd_workspace_size() is always enough), 256-byte aligned,
 *     owned by the caller; its contents need no
 *     initialisation and are undefined afterwards.
 *   - One pass enqueues three kernels on `stream` (per-chunk record, the two
 *     state recurrences, per-chunk gradients); no allocation, no
 *     synchronisation.  It keeps every chunk's state and state gradient in
 *     the workspace (about 108 KB per chunk and head with 16-bit inputs at
 *     K = V = 128).  A batch without cu_seqlens whose workspace holds fewer
 *     chunks runs in segments of as many chunks as it holds, last segment
 *     first: one forward call per earlier segment (gdn_fwd_launch, o into
 *     the workspace) leaves the fp32 state at each segment start, and each
 *     segment's backward passes the gradient of its initial state to the
 *     segment before.  The default sizes hold 256 chunks per sequence, so
 *     the workspace is bounded in T. */
typedef struct GdnBwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  const float* h0;           /* nullable */
  const void* d_o;           /* [B,T,H,V], unit stride along V (any b/t/h
                                strides, 0 included) */
  const float* d_final_state;/* nullable, [B,H,K,V] */
  void* dq;
  void* dk;
  void* dv;
  void* dg;
  void* dbeta;
  float* dh0;                /* nullable */
  void* workspace;
  /* strides in elements, (b, t, h) */
  int64_t q_stride[3];
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t g_stride[3];
  int64_t beta_stride[3];
  int64_t do_stride[3];
  int64_t dq_stride[3];
  int64_t dk_stride[3];
  int64_t dv_stride[3];
  int64_t dg_stride[3];
  int64_t dbeta_stride[3];
  /* strides in elements, (b, h, k, v) */
  int64_t h0_stride[4];
  int64_t dfs_stride[4];
  int64_t dh0_stride[4];
  int32_t B, T, H, K, V;
  float scale;
  int32_t qkv_dtype;         /* q, k, v and dq, dk, dv */
  int32_t g_dtype;           /* g and dg */
  int32_t beta_dtype;        /* beta and dbeta */
  int32_t do_dtype;
  const int64_t* cu_seqlens; /* nullable, as in GdnFwdParams */
  int64_t workspace_bytes;
} GdnBwdParams;

/* Bytes of workspace that gdn_bwd_launch needs for these sizes whatever
 * the dtypes (n_seq: the number of sequences with cu_seqlens, else 0); -1
 * if unsupported.  Without cu_seqlens, at most 256 chunks (8192 rows) per
 * sequence at a time. */
int64_t gdn_bwd_workspace_size(int B, int T, int H, int K, int V, int n_seq);

/* Bytes of workspace gdn_bwd_launch needs for exactly these params (their
 * sizes, dtypes, d_o alignment and cu_seqlens; pointers other than d_o and
 * cu_seqlens are not read); -1 if unsupported.  With 16-bit q, k, v and dO
 * of the same type, 4-byte aligned, the walks keep the chunk states in
 * fp16 and their records hold T and the gates only: about 55 % of
 * gdn_bwd_workspace_size at K = V = 128.  Without cu_seqlens, at most 256
 * chunks per sequence at a time. */
int64_t gdn_bwd_workspace_size_params(const GdnBwdParams* params);

/* As gdn_bwd_workspace_size_params, for segments of at most seg_chunks
 * chunks (>= 1; ignored with cu_seqlens).  No counterpart in the reference
 * (no backward there); for callers that trade time (one more forward pass
 * over all but the last segment) for memory. */
int64_t gdn_bwd_segment_workspace_size(const GdnBwdParams* params, int seg_chunks);

/* Enqueue the backward on `stream`; returns a GdnStatus / hipError_t. */
int gdn_bwd_launch(const GdnBwdParams* params, void* stream);

/* Human-readable text for a status code. */
const char* gdn_fwd_status_string(int status);

/* GDN_MI355X_ABI_VERSION of the built library. */
int gdn_fwd_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* GDN_MI355X_H */
