"""GPU parity of the fused input preparation (``gdn_prep``) against the oracle.

* q, k: ``x / sqrt(sum x^2 + eps)`` with the denominator rounded to x's
  dtype (gdn_ref.py:24-25).  The kernel sums squares in another order than
  torch, so an output may differ from the oracle's in the last place: fp16 /
  bf16 outputs by at most one unit (and > 99% are bit-equal), fp32 outputs
  by at most four.
* beta = sigmoid(x), g = logsigmoid(x): against the oracle's fp64 forms,
  within 4 fp32 ulps (relative 5e-7) of the fp64 value.
"""

import pytest
import torch

from oracle import gdn_oracle as ref

pytestmark = pytest.mark.gpu


def _ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of x's dtype at |x| (at least the smallest normal spacing)."""
    a = x.abs()
    up = torch.nextafter(a, torch.full_like(a, float("inf")))
    return (up - a).float()


def _check_rows(y_gpu, y_ref, name):
    """fp16 / bf16: within 1 ulp, > 99% bit-equal (the fp32 sum-order
    difference rarely survives the rounding to storage).  fp32: within 4 ulps
    (the sum's last-bit difference moves the quotient by up to 2)."""
    y_gpu, y_ref = y_gpu.cpu(), y_ref.cpu()
    diff = (y_gpu.float() - y_ref.float()).abs()
    lowp = y_ref.dtype != torch.float32
    tol = _ulp(y_ref) * (1 if lowp else 4)
    same = (y_gpu == y_ref).float().mean().item()
    print(f"[prep] {name}: bit-equal {same:.5f}, max diff / ulp "
          f"{(diff / _ulp(y_ref)).max().item():.2f}", flush=True)
    assert (diff <= tol).all(), name
    if lowp:
        assert same > 0.99, name


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("K", [32, 64, 128, 256])
def test_l2norm_rows(pkg, cuda, dtype, K):
    gen = torch.Generator().manual_seed(K)
    x = (2 * torch.randn(2, 37, 3, K, generator=gen)).to(dtype)
    x[0, 0, 0] = 0          # zero row: stays zero
    x[1, 5, 2] *= 1e-4      # |x|^2 comparable to eps
    y = pkg.l2norm(x.to(cuda))
    torch.cuda.synchronize()
    assert y.dtype == dtype and y.shape == x.shape
    _check_rows(y, ref.l2norm(x), f"{dtype} K={K}")
    assert torch.equal(y[0, 0, 0].cpu(), torch.zeros(K, dtype=dtype))


def test_prep_all_outputs_strided_inputs(pkg, cuda):
    """q and k as h-slices of a fused [B, T, 2H, K] projection (non-unit t / h
    strides), gates as strided fp16 / bf16 views."""
    B, T, H, K = 2, 300, 4, 128
    gen = torch.Generator().manual_seed(5)
    qk = torch.randn(B, T, 2 * H, K, generator=gen).half()
    q, k = qk[:, :, :H], qk[:, :, H:]
    graw = torch.randn(B, T, 2 * H, generator=gen)
    beta_in = graw[:, :, :H].half()                 # contiguous copy, fp16
    g_in = graw.to(torch.bfloat16)[:, :, H:]         # strided view, bf16
    d = lambda t: t.to(cuda)
    dq = d(qk)
    qn, kn, bo, go = pkg.gdn_prep(q=dq[:, :, :H], k=dq[:, :, H:], beta=d(beta_in),
                                  g=d(graw.to(torch.bfloat16))[:, :, H:])
    torch.cuda.synchronize()
    assert qn.is_contiguous() and kn.is_contiguous()
    _check_rows(qn, ref.l2norm(q), "q strided")
    _check_rows(kn, ref.l2norm(k), "k strided")
    assert bo.dtype == torch.float32 and go.dtype == torch.float32
    b64, g64 = ref.sigmoid(beta_in.float()), ref.logsigmoid(g_in.float())
    assert ((bo.cpu().double() - b64).abs() <= 5e-7 * b64.abs()).all()
    assert ((go.cpu().double() - g64).abs() <= 5e-7 * g64.abs() + 1e-30).all()


def test_gates_fp32_extremes(pkg, cuda):
    x = torch.cat([torch.linspace(-120, 120, 4801), torch.tensor([0.0, -1e-7, 1e-7, -88.0, 88.0])])
    n = x.numel()
    xb = x.reshape(1, n, 1)
    _, _, bo, go = pkg.gdn_prep(beta=xb.to(cuda), g=xb.to(cuda))
    torch.cuda.synchronize()
    b64, g64 = ref.sigmoid(xb), ref.logsigmoid(xb)
    bo, go = bo.cpu().double(), go.cpu().double()
    assert torch.isfinite(go).all()
    # sigmoid underflows to fp32 subnormals / zero for x < -87: absolute bound there
    assert ((bo - b64).abs() <= 5e-7 * b64.abs() + 1e-37).all()
    assert ((go - g64).abs() <= 5e-7 * g64.abs() + 1e-37).all()


def test_prep_in_place(pkg, cuda):
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(1, 64, 2, 64, generator=gen).half()
    b = torch.randn(1, 64, 2, generator=gen)
    dx, db = x.to(cuda), b.to(cuda)
    out = pkg.gdn_prep(q=dx, beta=db, inplace=True)
    torch.cuda.synchronize()
    assert out[0] is dx and out[2] is db
    _check_rows(dx, ref.l2norm(x), "in place")
    assert ((db.cpu().double() - ref.sigmoid(b)).abs() <= 5e-7).all()


def test_prep_full_size_row_norms(pkg, cuda):
    """cfg2 shapes (B2 T4096 H16 K128, fp16): every output row has norm 1
    to fp16 accuracy, and a sampled set of rows matches the oracle."""
    B, T, H, K = 2, 4096, 16, 128
    gen = torch.Generator(device="cpu").manual_seed(0)
    q = torch.randn(B, T, H, K, generator=gen).half()
    k = torch.randn(B, T, H, K, generator=gen).half()
    print("[prep] cfg2 row norms", flush=True)
    qn, kn, _, _ = pkg.gdn_prep(q=q.to(cuda), k=k.to(cuda))
    torch.cuda.synchronize()
    for y, x, name in ((qn, q, "q"), (kn, k, "k")):
        nrm = y.float().norm(dim=-1)
        assert (nrm - 1).abs().max().item() < 2e-3, name
        idx = torch.randint(0, T, (64,), generator=gen)
        _check_rows(y[:, idx].cpu(), ref.l2norm(x[:, idx]), f"cfg2 {name} sample")
