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


def _validate(q, k, v, g, beta, h0, chunk_size, block_v):
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
    if h0 is not None:
        if tuple(h0.shape) != (B, H, K, V):
            raise ValueError(f"h0 must be [B, H, K, V] = ({B}, {H}, {K}, {V}), got {tuple(h0.shape)}")
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
    dev = q.device
    if dev.type != "cuda":
        raise ValueError("gdn_fwd runs on a ROCm GPU: inputs must be on a cuda device "
                         f"(got {dev}); there is no CPU path")
    others = (k, v, g, beta) + ((h0,) if h0 is not None else ())
    if any(t.device != dev for t in others):
        raise ValueError("all inputs must be on the same device")
    if T > 0:
        for name, t in (("q", q), ("k", k), ("v", v)):
            _check_rows(t, name)
    return B, T, H, K, V


_KERNELS = {"auto": 0, "phased": _lib.FLAG_PHASED_KERNEL}

# Launch plans keyed by everything but the data pointers: shapes, strides,
# dtypes, devices and options.  A call whose signature was seen before skips
# the Python validation (it passed for that signature) and copies a
# prefilled parameter block, so the host cost per launch stays small next
# to the kernel.
_PLANS = {}
_PLANS_MAX = 256


class _Plan:
    __slots__ = ("shape_o", "shape_fs", "out_dtype", "fs_vk", "params")


def _signature(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype, kernel, fs_vk):
    hs = None if h0 is None else (h0.shape, h0.stride(), h0.dtype, h0.device)
    return (q.shape, q.stride(), q.dtype, q.device, k.shape, k.stride(), k.dtype, k.device,
            v.shape, v.stride(), v.dtype, v.device, g.shape, g.stride(), g.dtype, g.device,
            beta.shape, beta.stride(), beta.dtype, beta.device, hs, float(scale), chunk_size,
            block_v, output_dtype, kernel, fs_vk)


def _make_plan(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype, kernel, fs_vk):
    B, T, H, K, V = _validate(q, k, v, g, beta, h0, chunk_size, block_v)
    if kernel not in _KERNELS:
        raise ValueError(f"kernel={kernel!r} must be one of {sorted(_KERNELS)}")
    out_dtype = q.dtype if output_dtype is None else output_dtype
    if out_dtype not in _DTYPE_CODE:
        raise ValueError(f"output_dtype {out_dtype} not supported")
    plan = _Plan()
    plan.shape_o = (B, T, H, V)
    plan.shape_fs = (B, H, V, K) if fs_vk else (B, H, K, V)
    plan.out_dtype = out_dtype
    plan.fs_vk = fs_vk
    P = _lib.GdnFwdParams()
    P.q_stride[:] = q.stride()[:3]
    P.k_stride[:] = k.stride()[:3]
    P.v_stride[:] = v.stride()[:3]
    P.g_stride[:] = g.stride()
    P.beta_stride[:] = beta.stride()
    P.o_stride[:] = (T * H * V, H * V, V)          # o is allocated contiguous
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
    plan.params = bytes(P)
    return plan


def _run(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype, kernel, fs_vk):
    try:
        key = _signature(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype,
                         kernel, fs_vk)
        plan = _PLANS.get(key)
    except (AttributeError, TypeError):   # not tensors: _validate says which
        key, plan = None, None
    if plan is None:
        plan = _make_plan(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype,
                          kernel, fs_vk)
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
            kernel: str = "auto") -> Tuple[torch.Tensor, torch.Tensor]:
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
      kernel: ``"auto"`` runs the software-pipelined kernel where it applies
        (fp16/bf16, chunk 32, K in {64, 128}, block_v 16/32) and the
        phase-by-phase kernel elsewhere; ``"phased"`` forces the latter.

    Returns:
      ``o [B, T, H, V]`` and ``final_state [B, H, K, V]`` float32.

    Semantics are the reference's (gdn_ref.py:3-9): per step
    ``S = e^{g} S; u = beta (v - S^T k); S += k u^T; o = scale S^T q``.
    """
    return _run(q, k, v, g, beta, h0, scale, chunk_size, block_v, output_dtype, kernel, False)


def gdn_chunk_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                  g: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """The reference launcher's surface (gdn_triton.py:113-140).

    ``q, k [B,T,H,K]``, ``v [B,T,H,V]``, ``beta, g [B,T,H]`` (note: beta
    before g) -> ``o [B,T,H,V]`` in q.dtype and ``h_final [B,H,V,K]`` fp32
    (the reference's V x K state layout).  Zero initial state, scale 1.
    Any T is accepted: the trailing partial chunk is masked in-kernel, which
    equals the reference's zero padding (gdn_triton.py:121-125).
    """
    return _run(q, k, v, g, beta, None, 1.0, 32, None, None, "auto", True)


def auto_block_v(B: int, H: int, K: int, V: int, chunk_size: int = 32,
                 dtype: torch.dtype = torch.float16) -> int:
    """The V-slice width the launcher picks for this shape (-1: unsupported)."""
    return _lib.load_library().gdn_fwd_auto_block_v(B, H, K, V, chunk_size, _DTYPE_CODE[dtype])
