"""Python surface of the MI355X fused chunked GDN forward.

``gdn_fwd`` is the primary entry point, in the north-star argument order
``(q, k, v, g, beta, h0, scale) -> (o, final_state)`` with the K x V state
layout ``[B, H, K, V]``.  ``gdn_chunk_fwd`` reproduces the reference's own
launcher surface ``gdn_chunk_fwd(q, k, v, beta, g) -> (o, h_final [B,H,V,K])``
(gdn_triton.py:113-140).

Both validate on the host, allocate the outputs with ``torch.empty`` on the
inputs' device (as gdn_triton.py:126-127 does) and enqueue one kernel on the
current torch stream through the C ABI.  There is no CPU or PyTorch
fallback: without the HIP library or a ROCm device they raise.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _lib

_DTYPE_CODE = {
    torch.float32: _lib.DTYPE_F32,
    torch.float16: _lib.DTYPE_F16,
    torch.bfloat16: _lib.DTYPE_BF16,
}

SUPPORTED_K = (32, 64, 128, 256)
SUPPORTED_CHUNKS = (32, 64)
SUPPORTED_BLOCK_V = (16, 32, 64)


def _code(t: torch.Tensor, name: str) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise ValueError(f"{name}: dtype {t.dtype} not supported "
                         "(float32, float16, bfloat16)") from None


def _check_rows(t: torch.Tensor, name: str) -> None:
    """q/k/v rows are read with 16-byte vector loads."""
    if t.stride(-1) != 1:
        raise ValueError(f"{name}: the last dimension must be contiguous "
                         f"(stride {t.stride(-1)}); call .contiguous()")
    es = t.element_size()
    if t.data_ptr() % 16 != 0 or any((s * es) % 16 for s in t.stride()[:3]):
        raise ValueError(f"{name}: rows must be 16-byte aligned (data_ptr and "
                         f"b/t/h strides {t.stride()[:3]}); call .contiguous()")


def _validate(q, k, v, g, beta, h0, chunk_size, block_v, n_seq=None, check_device=True):
    """Checks the call; returns (units B, packed T, H, K, V).  With n_seq
    (cu_seqlens given) the tensors hold one packed batch of n_seq sequences."""
    for name, t in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k must be [B, T, H, K] and v [B, T, H, V]")
    B, T, H, K = q.shape
    V = v.shape[-1]
    if tuple(k.shape) != (B, T, H, K):
        raise ValueError(f"k shape {tuple(k.shape)} != q shape {tuple(q.shape)}")
    if tuple(v.shape[:3]) != (B, T, H):
        raise ValueError(f"v shape {tuple(v.shape)} does not match [B,T,H]=({B},{T},{H})")
    for name, t in (("g", g), ("beta", beta)):
        if tuple(t.shape) != (B, T, H):
            raise ValueError(f"{name} must be [B, T, H] = ({B}, {T}, {H}), got {tuple(t.shape)}")
    if n_seq is not None:
        if B != 1:
            raise ValueError(f"with cu_seqlens the inputs hold one packed batch: B must be 1, got {B}")
        B = n_seq
    if h0 is not None:
        if tuple(h0.shape) != (B, H, K, V):
            raise ValueError(f"h0 must be [N, H, K, V] = ({B}, {H}, {K}, {V}), got {tuple(h0.shape)}")
        if h0.dtype != torch.float32:
            raise ValueError(f"h0 must be float32, got {h0.dtype}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError(f"q, k, v must share a dtype (got {q.dtype}, {k.dtype}, {v.dtype})")
    _code(q, "q")
    _code(g, "g")
    _code(beta, "beta")
    if B <= 0 or H <= 0:
        raise ValueError(f"B and H must be positive (got B={B}, H={H})")
    if K not in SUPPORTED_K:
        raise ValueError(f"K={K} not supported (K in {SUPPORTED_K})")
    if V <= 0 or V % 16 != 0:
        raise ValueError(f"V={V} must be a positive multiple of 16")
    if chunk_size not in SUPPORTED_CHUNKS:
        raise ValueError(f"chunk_size={chunk_size} not supported {SUPPORTED_CHUNKS}")
    if block_v is not None and (block_v not in SUPPORTED_BLOCK_V or V % block_v):
        raise ValueError(f"block_v={block_v} must be one of {SUPPORTED_BLOCK_V} and divide V={V}")
    if check_device:
        _check_devices(q, k, v, g, beta, h0)
    if T > 0:
        for name, t in (("q", q), ("k", k), ("v", v)):
            _check_rows(t, name)
    return B, T, H, K, V


def _check_devices(q, *others):
    dev = q.device
    if dev.type != "cuda":
        raise ValueError("gdn_fwd runs on a ROCm GPU: inputs must be on a cuda device "
                         f"(got {dev}); there is no CPU path")
    others = tuple(t for t in others if t is not None)
    if any(t.device != dev for t in others):
        raise ValueError("all inputs must be on the same device")


_KERNELS = {"auto": 0, "phased": _lib.FLAG_PHASED_KERNEL, "fused": _lib.FLAG_FUSED_KERNEL}

# Launch plans keyed by everything but the data pointers: shapes, strides,
# dtypes, devices and options.  A call whose signature was seen before skips
# the Python validation (it passed for that signature) and copies a
# prefilled parameter block, so the host cost per launch stays small next
# to the kernel.
_PLANS = {}
_PLANS_MAX = 256


class _Plan:
    __slots__ = ("shape_o", "shape_fs", "out_dtype", "fs_vk", "o_hf", "params", "ws_bytes")


def _signature(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype, kernel, fs_vk,
               n_seq, o_hf, seg_chunks=None):
    hs = None if h0 is None else (h0.shape, h0.stride(), h0.dtype, h0.device)
    return (q.shape, q.stride(), q.dtype, q.device, k.shape, k.stride(), k.dtype, k.device,
            v.shape, v.stride(), v.dtype, v.device, g.shape, g.stride(), g.dtype, g.device,
            beta.shape, beta.stride(), beta.dtype, beta.device, hs, float(scale), chunk_size,
            block_v, output_dtype, kernel, fs_vk, n_seq, o_hf, seg_chunks)


def _make_plan(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype, kernel, fs_vk,
               n_seq, o_hf, seg_chunks=None):
    B, T, H, K, V = _validate(q, k, v, g, beta, h0, chunk_size, block_v, n_seq)
    if kernel not in _KERNELS:
        raise ValueError(f"kernel={kernel!r} must be one of {sorted(_KERNELS)}")
    out_dtype = q.dtype if output_dtype is None else output_dtype
    if out_dtype not in _DTYPE_CODE:
        raise ValueError(f"output_dtype {out_dtype} not supported")
    plan = _Plan()
    BO = q.shape[0]     # batches of o: 1 when packed
    plan.shape_o = (BO, H, T, V) if o_hf else (BO, T, H, V)
    plan.shape_fs = (B, H, V, K) if fs_vk else (B, H, K, V)
    plan.out_dtype = out_dtype
    plan.fs_vk = fs_vk
    plan.o_hf = o_hf
    P = _lib.GdnFwdParams()
    P.q_stride[:] = q.stride()[:3]
    P.k_stride[:] = k.stride()[:3]
    P.v_stride[:] = v.stride()[:3]
    P.g_stride[:] = g.stride()
    P.beta_stride[:] = beta.stride()
    if o_hf:    # o allocated contiguous [B, H, T, V], written through (b, t, h) strides
        P.o_stride[:] = (H * T * V, V, T * V)
    else:       # o allocated contiguous [B, T, H, V]
        P.o_stride[:] = (T * H * V, H * V, V)
    P.h0_stride[:] = h0.stride() if h0 is not None else (0, 0, 0, 0)
    if fs_vk:   # [B, H, V, K] tensor written through (b, h, k, v) strides
        P.fs_stride[:] = (H * V * K, V * K, 1, K)
    else:
        P.fs_stride[:] = (H * K * V, K * V, V, 1)
    P.B, P.T, P.H, P.K, P.V = B, T, H, K, V
    P.scale = float(scale)
    P.chunk_size = int(chunk_size)
    P.block_v = int(block_v or 0)
    P.qkv_dtype = _DTYPE_CODE[q.dtype]
    P.g_dtype = _DTYPE_CODE[g.dtype]
    P.beta_dtype = _DTYPE_CODE[beta.dtype]
    P.o_dtype = _DTYPE_CODE[out_dtype]
    P.flags = _KERNELS[kernel]
    # workspace bytes for these shapes (only whether cu_seqlens is set
    # matters to the size, not where it points)
    P.cu_seqlens = 1 if n_seq is not None else None
    lib = _lib.load_library()
    ws = lib.gdn_fwd_workspace_size(ctypes.byref(P))
    if ws < 0:
        raise ValueError(f"unsupported forward shape B={B} T={T} H={H} K={K} V={V}")
    if seg_chunks is not None and ws > 0:
        # the records of seg_chunks chunks per sequence (what a call of
        # seg_chunks * chunk_size rows takes): the call then runs in segments
        # of that many chunks (fewer records, more launches)
        if int(seg_chunks) < 1:
            raise ValueError(f"max_segment_chunks must be >= 1, got {seg_chunks}")
        P.T = min(T, chunk_size * int(seg_chunks))
        ws = lib.gdn_fwd_workspace_size(ctypes.byref(P))
        P.T = T
    P.cu_seqlens = None
    plan.ws_bytes = int(ws)
    plan.params = bytes(P)
    return plan


def _check_cu_seqlens(cu, T, dev):
    """Validates FLA-style packed-sequence offsets; returns (int64 tensor, N).
    Reads the offsets on the host (one small copy), as FLA's own varlen
    preparation does."""
    if not isinstance(cu, torch.Tensor) or cu.dim() != 1 or cu.numel() < 2:
        raise ValueError("cu_seqlens must be a 1-D tensor of N + 1 row offsets (N >= 1)")
    if cu.dtype not in (torch.int64, torch.int32):
        raise ValueError(f"cu_seqlens must be int64 or int32, got {cu.dtype}")
    if cu.device != dev:
        raise ValueError(f"cu_seqlens must be on {dev}, got {cu.device}")
    c = cu.tolist()
    if c[0] != 0 or c[-1] != T or any(b < a for a, b in zip(c, c[1:])):
        raise ValueError(f"cu_seqlens must rise from 0 to T={T} without decreasing, got {c}")
    if cu.dtype != torch.int64 or not cu.is_contiguous():
        cu = cu.to(torch.int64).contiguous()
    return cu, len(c) - 1


def _run(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype, kernel, fs_vk,
         cu_seqlens=None, o_hf=False, seg_chunks=None):
    n_seq = None
    if cu_seqlens is not None:
        if not isinstance(q, torch.Tensor) or q.dim() != 4:
            raise ValueError("q, k must be [B, T, H, K] and v [B, T, H, V]")
        cu_seqlens, n_seq = _check_cu_seqlens(cu_seqlens, q.shape[1], q.device)
    try:
        key = _signature(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype,
                         kernel, fs_vk, n_seq, o_hf, seg_chunks)
        plan = _PLANS.get(key)
    except (AttributeError, TypeError):   # not tensors: _validate says which
        key, plan = None, None
    if plan is None:
        plan = _make_plan(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype,
                          kernel, fs_vk, n_seq, o_hf, seg_chunks)
        if key is not None:
            if len(_PLANS) >= _PLANS_MAX:
                _PLANS.clear()
            _PLANS[key] = plan
    dev = q.device
    qp, kp, vp = q.data_ptr(), k.data_ptr(), v.data_ptr()
    if plan.shape_o[1] > 0 and (qp | kp | vp) & 15:
        for name, t in (("q", q), ("k", k), ("v", v)):
            _check_rows(t, name)
    o = torch.empty(plan.shape_o, dtype=plan.out_dtype, device=dev)
    fs = torch.empty(plan.shape_fs, dtype=torch.float32, device=dev)
    P = _lib.GdnFwdParams.from_buffer_copy(plan.params)
    P.q, P.k, P.v = qp, kp, vp
    P.g, P.beta = g.data_ptr(), beta.data_ptr()
    P.h0 = h0.data_ptr() if h0 is not None else None
    P.o, P.final_state = o.data_ptr(), fs.data_ptr()
    P.cu_seqlens = cu_seqlens.data_ptr() if cu_seqlens is not None else None
    ws = None   # released when this call returns: later work on the stream is ordered after it
    if plan.ws_bytes > 0:
        ws = torch.empty(plan.ws_bytes, dtype=torch.uint8, device=dev)
        P.workspace, P.workspace_bytes = ws.data_ptr(), plan.ws_bytes
    lib = _lib.load_library()
    if dev.index == torch.cuda.current_device():
        status = lib.gdn_fwd_launch(ctypes.byref(P), torch.cuda.current_stream(dev).cuda_stream)
    else:
        with torch.cuda.device(dev):
            status = lib.gdn_fwd_launch(ctypes.byref(P), torch.cuda.current_stream(dev).cuda_stream)
    if status != 0:
        raise RuntimeError(f"gdn_fwd_launch failed ({status}): {_lib.status_string(status)}")
    return o, fs


def gdn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
            beta: torch.Tensor, h0: Optional[torch.Tensor] = None, scale: float = 1.0,
            chunk_size: int = 32, *, block_v: Optional[int] = None,
            output_dtype: Optional[torch.dtype] = None,
            kernel: str = "auto",
            cu_seqlens: Optional[torch.Tensor] = None,
            max_segment_chunks: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused chunked Gated DeltaNet forward on an MI355X.

    Args:
      q, k: ``[B, T, H, K]``; v: ``[B, T, H, V]`` -- float16, bfloat16 or
        float32 (one dtype for all three), last dim contiguous.
      g: ``[B, T, H]`` log-decay gates (``gamma_t = e^{g_t}``).
      beta: ``[B, T, H]`` write strengths.  g and beta may be float32,
        float16 or bfloat16, any strides.
      h0: optional ``[B, H, K, V]`` float32 initial state (K x V form).
      scale: output scale, ``o_t = scale * S_t^T q_t``.
      chunk_size: 32 or 64.
      block_v: V columns per workgroup (16, 32, 64); None picks one.
      output_dtype: dtype of ``o``; defaults to ``q.dtype`` (as the
        reference, gdn_triton.py:126).
      kernel: ``"auto"`` picks per shape: for fp16 or bf16 with chunk 32
        and K in {64, 128}, per-chunk records then the scan (two launches
        per segment, a workspace of records; bf16 records also carry the
        chunk's k rows in fp16); the phase-by-phase kernel elsewhere.  ``"fused"``
        forces the fused pipelined kernel (no workspace) where it applies,
        ``"phased"`` the phase-by-phase kernel.
      cu_seqlens: optional int64 ``[N + 1]`` row offsets: N sequences
        packed along t of a batch of one (B = 1); sequence i is rows
        ``cu_seqlens[i]:cu_seqlens[i+1]`` with its own ``h0[i]`` and
        ``final_state[i]`` (h0 and final_state are then ``[N, H, K, V]``).
      max_segment_chunks: for the two-launch paths, the records of at most
        this many chunks per sequence are held at once; a longer sequence
        runs as several segments (default: 256 chunks of 32 rows, 64 chunks
        of 64 rows).

    Returns:
      ``o [B, T, H, V]`` and ``final_state [B, H, K, V]`` float32.  When an
      input requires grad (and grad mode is on) both outputs are
      differentiable; the backward runs ``gdn_bwd`` (K in {32, 64, 128}).

    Semantics are the reference's (gdn_ref.py:3-9): per step
    ``S = e^{g} S; u = beta (v - S^T k); S += k u^T; o = scale S^T q``.
    """
    if _needs_grad(q, k, v, g, beta, h0):
        return _GdnFunction.apply(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype,
                                  kernel, False, cu_seqlens, False, max_segment_chunks)
    return _run(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype, kernel, False,
                cu_seqlens, False, max_segment_chunks)


def gdn_chunk_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                  g: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """The reference launcher's surface (gdn_triton.py:113-140).

    ``q, k [B,T,H,K]``, ``v [B,T,H,V]``, ``beta, g [B,T,H]`` (note: beta
    before g) -> ``o [B,T,H,V]`` in q.dtype and ``h_final [B,H,V,K]`` fp32
    (the reference's V x K state layout).  Zero initial state, scale 1.
    Any T is accepted: the trailing partial chunk is masked in-kernel, which
    equals the reference's zero padding (gdn_triton.py:121-125).
    """
    if _needs_grad(q, k, v, g, beta):
        return _GdnFunction.apply(q, k, v, g, beta, None, 1.0, 32, None, None, "auto", True,
                                  None, False)
    return _run(q, k, v, g, beta, None, 1.0, 32, None, None, "auto", True)


def auto_block_v(B: int, H: int, K: int, V: int, chunk_size: int = 32,
                 dtype: torch.dtype = torch.float16) -> int:
    """The V-slice width the launcher picks for this shape (-1: unsupported)."""
    return _lib.load_library().gdn_fwd_auto_block_v(B, H, K, V, chunk_size, _DTYPE_CODE[dtype])


# ---------------------------------------------------------------------------
# input preparation (the step before the path)
# ---------------------------------------------------------------------------

def _bth_strides(t: torch.Tensor):
    return t.stride()[:3]


def _prep_plan(q, k, beta, g, eps, out_gate_dtype, inplace):
    """Validates a preparation call and builds its parameter block (pointers
    left zero); returns (params bytes, output specs)."""
    rows = [t for t in (q, k) if t is not None]
    gts = [t for t in (beta, g) if t is not None]
    ref = rows[0] if rows else gts[0]
    if not isinstance(ref, torch.Tensor):
        raise TypeError("gdn_prep inputs must be torch tensors")
    dev = ref.device
    if rows:
        if q is not None and k is not None and (q.shape != k.shape or q.dtype != k.dtype):
            raise ValueError(f"q and k must share shape and dtype ({tuple(q.shape)} {q.dtype} vs "
                             f"{tuple(k.shape)} {k.dtype})")
        if ref.dim() != 4:
            raise ValueError("q, k must be [B, T, H, K]")
        B, T, H, K = ref.shape
        if K not in SUPPORTED_K:
            raise ValueError(f"K={K} not supported (K in {SUPPORTED_K})")
    else:
        if ref.dim() != 3:
            raise ValueError("beta, g must be [B, T, H]")
        B, T, H = ref.shape
        K = 0
    for name, t in (("beta", beta), ("g", g)):
        if t is not None and tuple(t.shape) != (B, T, H):
            raise ValueError(f"{name} must be [B, T, H] = ({B}, {T}, {H}), got {tuple(t.shape)}")
    for t in rows + gts:
        _code(t, "input")
        if t.device != dev:
            raise ValueError("all inputs must be on the same device")
    if out_gate_dtype not in _DTYPE_CODE:
        raise ValueError(f"out_gate_dtype {out_gate_dtype} not supported")
    if dev.type != "cuda":
        raise ValueError(f"gdn_prep runs on a ROCm GPU (got {dev}); there is no CPU path")
    P = _lib.GdnPrepParams()
    P.B, P.T, P.H, P.K = B, T, H, K
    P.eps = float(eps)
    specs = []   # per output: None, or (shape, dtype) of a new contiguous tensor
    for name, t in (("q", q), ("k", k)):
        if t is None:
            specs.append(None)
            continue
        if T > 0:
            _check_rows(t, name)
        getattr(P, f"{name}_in_stride")[:] = _bth_strides(t)
        getattr(P, f"{name}_out_stride")[:] = (_bth_strides(t) if inplace else
                                               (T * H * K, H * K, K))
        P.qk_dtype = _DTYPE_CODE[t.dtype]
        specs.append((tuple(t.shape), t.dtype))
    for name, t in (("beta", beta), ("g", g)):
        if t is None:
            specs.append(None)
            continue
        if inplace and t.dtype != out_gate_dtype:
            raise ValueError(f"inplace needs {name} in out_gate_dtype {out_gate_dtype}")
        getattr(P, f"{name}_in_stride")[:] = t.stride()
        getattr(P, f"{name}_out_stride")[:] = t.stride() if inplace else (T * H, H, 1)
        setattr(P, f"{name}_in_dtype", _DTYPE_CODE[t.dtype])
        setattr(P, f"{name}_out_dtype", _DTYPE_CODE[out_gate_dtype])
        specs.append((tuple(t.shape), out_gate_dtype))
    return bytes(P), specs


_PREP_PLANS = {}


def gdn_prep(q: Optional[torch.Tensor] = None, k: Optional[torch.Tensor] = None,
             beta: Optional[torch.Tensor] = None, g: Optional[torch.Tensor] = None,
             eps: float = 1e-6, *, out_gate_dtype: torch.dtype = torch.float32,
             inplace: bool = False):
    """One fused launch preparing the forward's inputs.

    * ``q, k [B, T, H, K]`` -> ``x / sqrt(sum(x^2) + eps)`` over K, the sum in
      fp32 and the denominator rounded to x's dtype before the division, as
      the reference's ``_l2norm`` (gdn_ref.py:24-25);
    * ``beta [B, T, H]`` (logits) -> ``sigmoid(beta)``;
    * ``g [B, T, H]`` (logits) -> ``logsigmoid(g)``;

    Any argument may be None (its result is None).  Outputs are new
    contiguous tensors (q/k in their dtype, gates in ``out_gate_dtype``), or
    the inputs themselves when ``inplace``.  Launch plans are cached by
    shapes, strides and dtypes, as for ``gdn_fwd``.
    """
    ins = (q, k, beta, g)
    if all(t is None for t in ins):
        return None, None, None, None
    try:
        key = tuple(None if t is None else (t.shape, t.stride(), t.dtype, t.device) for t in ins)
        key += (float(eps), out_gate_dtype, inplace)
        plan = _PREP_PLANS.get(key)
    except (AttributeError, TypeError):
        key, plan = None, None
    if plan is None:
        plan = _prep_plan(q, k, beta, g, eps, out_gate_dtype, inplace)
        if key is not None:
            if len(_PREP_PLANS) >= _PLANS_MAX:
                _PREP_PLANS.clear()
            _PREP_PLANS[key] = plan
    params, specs = plan
    rows = [t for t in (q, k) if t is not None]
    if rows and rows[0].shape[1] > 0 and any(t.data_ptr() & 15 for t in rows):
        for name, t in (("q", q), ("k", k)):
            if t is not None:
                _check_rows(t, name)
    dev = next(t for t in ins if t is not None).device
    outs = tuple(None if sp is None else (t if inplace else torch.empty(sp[0], dtype=sp[1], device=dev))
                 for t, sp in zip(ins, specs))
    P = _lib.GdnPrepParams.from_buffer_copy(params)
    for name, t, o in zip(("q", "k", "beta", "g"), ins, outs):
        if t is not None:
            setattr(P, f"{name}_in", t.data_ptr())
            setattr(P, f"{name}_out", o.data_ptr())
    lib = _lib.load_library()
    if dev.index == torch.cuda.current_device():
        status = lib.gdn_prep_launch(ctypes.byref(P), torch.cuda.current_stream(dev).cuda_stream)
    else:
        with torch.cuda.device(dev):
            status = lib.gdn_prep_launch(ctypes.byref(P), torch.cuda.current_stream(dev).cuda_stream)
    if status != 0:
        raise RuntimeError(f"gdn_prep_launch failed ({status}): {_lib.status_string(status)}")
    return outs


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``x / sqrt(sum(x^2) + eps)`` over the last dim on the GPU
    (gdn_ref.py:24-25), for ``[B, T, H, K]`` tensors."""
    return gdn_prep(q=x, eps=eps)[0]


# ---------------------------------------------------------------------------
# FLA's keyword surface
# ---------------------------------------------------------------------------

def chunk_gated_delta_rule(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                           beta: torch.Tensor, scale: Optional[float] = None,
                           initial_state: Optional[torch.Tensor] = None,
                           output_final_state: bool = False,
                           cu_seqlens: Optional[torch.Tensor] = None,
                           head_first: bool = False,
                           use_qk_l2norm_in_kernel: bool = False):
    """Drop-in for FLA's ``chunk_gated_delta_rule`` (FLA 0.6.0, the comparator
    the reference calls by keyword at bench_gdn.py:169-172 and
    bench_zoo.py:38-42), on this build's kernel.

    Args follow FLA: ``q, k [B, T, H, K]``, ``v [B, T, H, V]``, ``g, beta
    [B, T, H]`` (``[B, H, T, *]`` with ``head_first``); ``scale`` defaults to
    ``K ** -0.5``; ``initial_state [N, H, K, V]``; ``cu_seqlens`` int64
    ``[N + 1]`` offsets of N sequences packed along t (B = 1);
    ``use_qk_l2norm_in_kernel`` L2-normalises q and k first (one fused
    preparation launch).

    Returns ``(o, final_state)``: ``o`` like ``v`` (``[B, H, T, V]`` with
    ``head_first``) in q's dtype, ``final_state [N, H, K, V]`` float32 when
    ``output_final_state`` else None.
    """
    for name, t in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
    if head_first:
        if q.dim() != 4 or k.dim() != 4 or v.dim() != 4 or g.dim() != 3 or beta.dim() != 3:
            raise ValueError("head_first: q, k [B, H, T, K], v [B, H, T, V], g, beta [B, H, T]")
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        g, beta = g.transpose(1, 2), beta.transpose(1, 2)
    if scale is None:
        scale = q.shape[-1] ** -0.5
    if use_qk_l2norm_in_kernel:
        if _needs_grad(q, k):
            raise NotImplementedError("use_qk_l2norm_in_kernel with gradients through q, k is not "
                                      "supported: normalise with gdn_prep / l2norm first")
        q, k, _, _ = gdn_prep(q=q, k=k)
    h0 = initial_state
    if h0 is not None and h0.dtype != torch.float32:
        h0 = h0.float()
    if _needs_grad(q, k, v, g, beta, h0):
        o, fs = _GdnFunction.apply(q, k, v, g, beta, h0, scale, 32, None, None, "auto", False,
                                   cu_seqlens, head_first)
    else:
        o, fs = _run(q, k, v, g, beta, h0, scale, 32, None, None, "auto", False, cu_seqlens,
                     head_first)
    return o, (fs if output_final_state else None)


# ---------------------------------------------------------------------------
# backward
# ---------------------------------------------------------------------------

BWD_SUPPORTED_K = (32, 64, 128)


def gdn_bwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
            beta: torch.Tensor, h0: Optional[torch.Tensor], do: torch.Tensor,
            dfinal: Optional[torch.Tensor] = None, scale: float = 1.0,
            cu_seqlens: Optional[torch.Tensor] = None, need_dh0: bool = True,
            max_segment_chunks: Optional[int] = None):
    """Gradients of ``gdn_fwd`` (the recurrence gdn_ref.py:3-9) with respect to
    ``q, k, v, g, beta, h0``, given ``do`` (the gradient of ``o``, ``[B,T,H,V]``)
    and ``dfinal`` (the gradient of ``final_state``, ``[B,H,K,V]`` fp32, or
    None for zero).

    Returns ``(dq, dk, dv, dg, dbeta, dh0)`` in the inputs' dtypes (``dh0``
    fp32, None unless ``need_dh0``).  K in {32, 64, 128}, V a multiple of 16;
    same strides, dtypes and ``cu_seqlens`` convention as the forward.  One
    call enqueues the backward's three kernels on the current stream; the
    workspace (per-chunk records, chunk-start states and their gradients,
    u and du) is allocated here and released when the call returns.  It
    holds at most ``max_segment_chunks`` chunks of 32 rows per sequence
    (default 256): a longer batch runs in segments, with one forward pass
    over all but the last segment for the states at their starts
    (``gdn_bwd_launch``).  Packed sequences run in one pass.
    """
    n_seq = None
    if cu_seqlens is not None:
        cu_seqlens, n_seq = _check_cu_seqlens(cu_seqlens, q.shape[1], q.device)
    B, T, H, K, V = _validate(q, k, v, g, beta, h0, 32, None, n_seq, check_device=False)
    if K not in BWD_SUPPORTED_K:
        raise ValueError(f"K={K} not supported by the backward (K in {BWD_SUPPORTED_K})")
    if not isinstance(do, torch.Tensor) or tuple(do.shape) != tuple(v.shape):
        raise ValueError(f"do must have o's shape {tuple(v.shape)}")
    _code(do, "do")
    if dfinal is not None:
        if tuple(dfinal.shape) != (B, H, K, V) or dfinal.dtype != torch.float32:
            raise ValueError(f"dfinal must be float32 [{B}, {H}, {K}, {V}]")
    _check_devices(q, k, v, g, beta, h0, do, dfinal)
    # The kernels index dO rows by their (b, t, h) strides with a unit step
    # along V.  autograd may hand over any layout, e.g. the stride-0 expansion
    # of a scalar for o.sum().backward(): give the kernels a dense copy then.
    if do.stride(-1) != 1:
        do = do.contiguous()
    dev = q.device
    lib = _lib.load_library()
    dq = torch.empty(q.shape, dtype=q.dtype, device=dev)
    dk = torch.empty(k.shape, dtype=k.dtype, device=dev)
    dv = torch.empty(v.shape, dtype=v.dtype, device=dev)
    dg = torch.empty(g.shape, dtype=g.dtype, device=dev)
    dbeta = torch.empty(beta.shape, dtype=beta.dtype, device=dev)
    dh0 = torch.empty(B, H, K, V, dtype=torch.float32, device=dev) if need_dh0 else None
    P = _lib.GdnBwdParams()
    P.q, P.k, P.v, P.g, P.beta = q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr()
    P.h0 = h0.data_ptr() if h0 is not None else None
    P.d_o = do.data_ptr()
    P.d_final_state = dfinal.data_ptr() if dfinal is not None else None
    P.dq, P.dk, P.dv, P.dg, P.dbeta = dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dg.data_ptr(), dbeta.data_ptr()
    P.dh0 = dh0.data_ptr() if dh0 is not None else None
    for name, t in (("q", q), ("k", k), ("v", v), ("do", do), ("dq", dq), ("dk", dk), ("dv", dv)):
        getattr(P, f"{name}_stride")[:] = t.stride()[:3]
    for name, t in (("g", g), ("beta", beta), ("dg", dg), ("dbeta", dbeta)):
        getattr(P, f"{name}_stride")[:] = t.stride()
    P.h0_stride[:] = h0.stride() if h0 is not None else (0, 0, 0, 0)
    P.dfs_stride[:] = dfinal.stride() if dfinal is not None else (0, 0, 0, 0)
    P.dh0_stride[:] = dh0.stride() if dh0 is not None else (0, 0, 0, 0)
    P.B, P.T, P.H, P.K, P.V = B, T, H, K, V
    P.scale = float(scale)
    P.qkv_dtype = _DTYPE_CODE[q.dtype]
    P.g_dtype = _DTYPE_CODE[g.dtype]
    P.beta_dtype = _DTYPE_CODE[beta.dtype]
    P.do_dtype = _DTYPE_CODE[do.dtype]
    P.cu_seqlens = cu_seqlens.data_ptr() if cu_seqlens is not None else None
    # the workspace this call's path takes (the 16-bit walks need less)
    if max_segment_chunks is None:
        ws_bytes = lib.gdn_bwd_workspace_size_params(ctypes.byref(P))
    else:
        if int(max_segment_chunks) < 1:
            raise ValueError(f"max_segment_chunks must be >= 1, got {max_segment_chunks}")
        ws_bytes = lib.gdn_bwd_segment_workspace_size(ctypes.byref(P), int(max_segment_chunks))
    if ws_bytes < 0:
        raise ValueError(f"backward does not support B={B} T={T} H={H} K={K} V={V}")
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    P.workspace, P.workspace_bytes = ws.data_ptr(), ws.numel()
    with torch.cuda.device(dev):
        status = lib.gdn_bwd_launch(ctypes.byref(P), torch.cuda.current_stream(dev).cuda_stream)
    if status != 0:
        raise RuntimeError(f"gdn_bwd_launch failed ({status}): {_lib.status_string(status)}")
    return dq, dk, dv, dg, dbeta, dh0


class _GdnFunction(torch.autograd.Function):
    """``_run`` with the HIP backward: o, final_state differentiable in
    q, k, v, g, beta and h0."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype, kernel,
                fs_vk, cu_seqlens, o_hf, seg_chunks=None):
        o, fs = _run(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype, kernel,
                     fs_vk, cu_seqlens, o_hf, seg_chunks)
        ctx.save_for_backward(q, k, v, g, beta, h0, cu_seqlens)
        ctx.scale, ctx.fs_vk, ctx.o_hf = scale, fs_vk, o_hf
        return o, fs

    @staticmethod
    def backward(ctx, do, dfs):
        q, k, v, g, beta, h0, cu = ctx.saved_tensors
        if do is None:
            shape = (v.shape[0], v.shape[2], v.shape[1], v.shape[3]) if ctx.o_hf else v.shape
            do = torch.zeros(shape, dtype=q.dtype, device=q.device)
        do_bthv = do.transpose(1, 2) if ctx.o_hf else do
        dfs_kv = None if dfs is None else (dfs.transpose(2, 3) if ctx.fs_vk else dfs)
        if dfs_kv is not None and dfs_kv.dtype != torch.float32:
            dfs_kv = dfs_kv.float()
        need_dh0 = h0 is not None and ctx.needs_input_grad[5]
        dq, dk, dv, dg, dbeta, dh0 = gdn_bwd(q, k, v, g, beta, h0, do_bthv, dfs_kv, ctx.scale,
                                             cu_seqlens=cu, need_dh0=need_dh0)
        return dq, dk, dv, dg, dbeta, dh0, None, None, None, None, None, None, None, None, None


def _needs_grad(*ts) -> bool:
    return torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad
                                           for t in ts)
